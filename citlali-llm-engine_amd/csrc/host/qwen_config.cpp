// qwen_config.cpp -- QwenConfig from GGUF metadata.
//
// Key names, defaults, fallbacks and checks follow the reference's
// src/model/qwen_config.cpp:59-151 in the same order: sizes are read as
// u32 through get_u64 (so u64/u32/i64/i32 all work, a negative one counts
// as absent), floats through get_f32.
#include "citlali/model/qwen_config.h"

#include "citlali/common.h"

namespace citlali::model {

namespace {

uint32_t size_key(const io::GgufFile& g, const std::string& arch, const char* name, uint32_t fallback = 0) {
    return static_cast<uint32_t>(g.get_u64(arch + "." + name, fallback));
}

float float_key(const io::GgufFile& g, const std::string& arch, const char* name, float fallback) {
    return g.get_f32(arch + "." + name, fallback);
}

// rows of blk.0.<weight> per head, or 0 when the tensor or the split is missing
uint32_t rows_per_head(const io::GgufFile& g, const char* weight, uint32_t heads) {
    const io::GgufTensorInfo* t = g.find_tensor(std::string("blk.0.") + weight);
    if (t == nullptr || t->dims.size() < 2 || t->dims[1] % heads != 0) return 0;
    return static_cast<uint32_t>(t->dims[1] / heads);
}

}  // namespace

QwenConfig QwenConfig::from_gguf(const io::GgufFile& g) {
    QwenConfig c;
    c.architecture = g.get_string("general.architecture", "qwen3");
    require(c.architecture.find("qwen") != std::string::npos,
            "Only Qwen/Qwen3 dense GGUF is supported in this engine");
    const std::string& a = c.architecture;
    c.vocab_size = static_cast<uint32_t>(g.get_string_array("tokenizer.ggml.tokens").size());
    c.context_length = size_key(g, a, "context_length", 2048);
    c.embedding_length = size_key(g, a, "embedding_length");
    c.block_count = size_key(g, a, "block_count");
    c.feed_forward_length = size_key(g, a, "feed_forward_length");
    c.head_count = size_key(g, a, "attention.head_count");
    c.head_count_kv = size_key(g, a, "attention.head_count_kv", c.head_count);
    c.head_dim = size_key(g, a, "attention.key_length");
    c.value_dim = size_key(g, a, "attention.value_length");
    c.rms_norm_eps = float_key(g, a, "attention.layer_norm_rms_epsilon", 1e-6f);
    c.rope_theta = float_key(g, a, "rope.freq_base", 1000000.0f);

    // files that name their keys qwen2.* under another architecture string
    const std::string q2 = "qwen2";
    if (c.embedding_length == 0) c.embedding_length = size_key(g, q2, "embedding_length");
    if (c.block_count == 0) c.block_count = size_key(g, q2, "block_count");
    if (c.feed_forward_length == 0) c.feed_forward_length = size_key(g, q2, "feed_forward_length");
    if (c.head_count == 0) c.head_count = size_key(g, q2, "attention.head_count");
    if (c.head_count_kv == 0) c.head_count_kv = size_key(g, q2, "attention.head_count_kv", c.head_count);
    if (c.head_dim == 0) c.head_dim = size_key(g, q2, "attention.key_length");
    if (c.value_dim == 0) c.value_dim = size_key(g, q2, "attention.value_length");

    require(c.vocab_size > 0, "failed to read vocab size from GGUF");
    require(c.embedding_length > 0, "failed to read embedding_length from GGUF");
    require(c.block_count > 0, "failed to read block_count from GGUF");
    require(c.feed_forward_length > 0, "failed to read feed_forward_length from GGUF");
    require(c.head_count > 0, "failed to read attention.head_count from GGUF");
    require(c.head_count_kv > 0, "failed to read attention.head_count_kv from GGUF");
    if (c.head_dim == 0) c.head_dim = rows_per_head(g, "attn_q.weight", c.head_count);
    if (c.value_dim == 0) c.value_dim = rows_per_head(g, "attn_v.weight", c.head_count_kv);
    if (c.head_dim == 0) {
        require(c.embedding_length % c.head_count == 0,
                "embedding_length must be divisible by head_count when attention.key_length is absent");
        c.head_dim = c.embedding_length / c.head_count;
    }
    if (c.value_dim == 0) c.value_dim = c.head_dim;
    require(c.head_dim > 0, "failed to read or derive attention.key_length/head_dim from GGUF");
    require(c.value_dim == c.head_dim,
            "this minimal attention path currently requires attention.value_length == attention.key_length");
    return c;
}

}  // namespace citlali::model
