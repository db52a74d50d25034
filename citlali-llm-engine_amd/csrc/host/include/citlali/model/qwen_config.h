// citlali/model/qwen_config.h -- model hyper-parameters.
//
// Same fields and defaults as the reference's QwenConfig
// (include/citlali/model/qwen_config.h:8-23); reading them from GGUF
// metadata (QwenConfig::from_gguf) belongs to the loader, outside this path.
#pragma once

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
};

}  // namespace citlali::model
