// citlali/model/qwen_config.h -- model hyper-parameters.
//
// Same fields and defaults as the reference's QwenConfig
// (include/citlali/model/qwen_config.h:8-25), read from GGUF metadata by
// from_gguf (src/model/qwen_config.cpp:59-151).
#pragma once

#include "citlali/io/gguf_reader.h"

#include <cstdint>
#include <string>

namespace citlali::model {

struct QwenConfig {
    std::string architecture;
    uint32_t vocab_size = 0;
    uint32_t context_length = 0;
    uint32_t embedding_length = 0;   // hidden size
    uint32_t block_count = 0;        // layers
    uint32_t feed_forward_length = 0;
    uint32_t head_count = 0;
    uint32_t head_count_kv = 0;
    uint32_t head_dim = 0;
    uint32_t value_dim = 0;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 1000000.0f;

    // `<arch>.*` keys (arch = general.architecture, default "qwen3", must
    // contain "qwen"), then `qwen2.*` for sizes still 0; vocab_size = the
    // length of tokenizer.ggml.tokens.  head_dim / value_dim missing from the
    // metadata come from blk.0.attn_q / attn_v rows per head, else
    // embedding_length / head_count.  Throws citlali::Error for a size it
    // cannot find or value_dim != head_dim.
    static QwenConfig from_gguf(const io::GgufFile& gguf);
};

}  // namespace citlali::model
