// kernels.cpp -- the compute:: launchers over the C ABI.  Each forwards its
// arguments unchanged (reference kernels.cu:659-876 launchers) and turns a
// non-zero status into citlali::Error.
#include "citlali/compute/hip/kernels.h"

#include "citlali/compute/hip/hip_check.h"

namespace citlali::compute {

void cuda_zero(void* data, std::size_t bytes) { CITLALI_HIP_CHECK(citlali_hip_zero(data, bytes)); }
void device_zero(void* data, std::size_t bytes) { cuda_zero(data, bytes); }

void launch_embed(const uint16_t* embedding, int32_t token_id, uint16_t* out, int hidden) {
    CITLALI_HIP_CHECK(citlali_hip_embed(embedding, token_id, out, hidden));
}

void launch_copy(const uint16_t* input, uint16_t* output, int n) {
    CITLALI_HIP_CHECK(citlali_hip_copy(input, output, n));
}

void launch_add_inplace(uint16_t* target, const uint16_t* delta, int n) {
    CITLALI_HIP_CHECK(citlali_hip_add_inplace(target, delta, n));
}

void launch_add_bias_inplace(uint16_t* target, const uint16_t* bias, int n) {
    CITLALI_HIP_CHECK(citlali_hip_add_bias_inplace(target, bias, n));
}

void launch_rms_norm(const uint16_t* input, const uint16_t* weight, uint16_t* output, int n, float eps) {
    CITLALI_HIP_CHECK(citlali_hip_rms_norm(input, weight, output, n, eps));
}

void launch_rms_norm_heads(const uint16_t* input, const uint16_t* weight, uint16_t* output, int heads,
                           int head_dim, float eps) {
    CITLALI_HIP_CHECK(citlali_hip_rms_norm_heads(input, weight, output, heads, head_dim, eps));
}

void launch_matvec_fp16(const uint16_t* weight, const uint16_t* input, uint16_t* output, int in_features,
                        int out_features) {
    CITLALI_HIP_CHECK(citlali_hip_matvec_fp16(weight, input, output, in_features, out_features));
}

void launch_matvec_fp16_to_float(const uint16_t* weight, const uint16_t* input, float* output, int in_features,
                                 int out_features) {
    CITLALI_HIP_CHECK(citlali_hip_matvec_fp16_to_float(weight, input, output, in_features, out_features));
}

void launch_matvec_q4k(const uint8_t* weight, const uint16_t* input, uint16_t* output, int in_features,
                       int out_features) {
    CITLALI_HIP_CHECK(citlali_hip_matvec_q4k(weight, input, output, in_features, out_features));
}

void launch_matvec_q6k(const uint8_t* weight, const uint16_t* input, uint16_t* output, int in_features,
                       int out_features) {
    CITLALI_HIP_CHECK(citlali_hip_matvec_q6k(weight, input, output, in_features, out_features));
}

void launch_matvec_q6k_to_float(const uint8_t* weight, const uint16_t* input, float* output, int in_features,
                                int out_features) {
    CITLALI_HIP_CHECK(citlali_hip_matvec_q6k_to_float(weight, input, output, in_features, out_features));
}

void launch_embed_q6k(const uint8_t* embedding, int32_t token_id, uint16_t* output, int hidden) {
    CITLALI_HIP_CHECK(citlali_hip_embed_q6k(embedding, token_id, output, hidden));
}

void launch_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* output, int n) {
    CITLALI_HIP_CHECK(citlali_hip_swiglu(gate, up, output, n));
}

void launch_rope(uint16_t* data, int heads, int head_dim, int position, float theta) {
    CITLALI_HIP_CHECK(citlali_hip_rope(data, heads, head_dim, position, theta));
}

void launch_store_kv(const uint16_t* k, const uint16_t* v, uint16_t* k_cache, uint16_t* v_cache, int position,
                     int kv_size) {
    CITLALI_HIP_CHECK(citlali_hip_store_kv(k, v, k_cache, v_cache, position, kv_size));
}

void launch_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* scores,
                      uint16_t* output, int position, int max_context, int heads, int kv_heads, int head_dim) {
    CITLALI_HIP_CHECK(citlali_hip_attention(q, k_cache, v_cache, scores, output, position, max_context, heads,
                                            kv_heads, head_dim));
}

void launch_add_rms_norm(uint16_t* x, const uint16_t* delta, const uint16_t* weight, uint16_t* output, int n,
                         float eps) {
    CITLALI_HIP_CHECK(citlali_hip_add_rms_norm(x, delta, weight, output, n, eps));
}

void launch_qk_norm_rope_store(uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                               const uint16_t* k_norm, int heads, int kv_heads, int head_dim, int position,
                               float theta, float eps, uint16_t* k_cache, uint16_t* v_cache) {
    CITLALI_HIP_CHECK(citlali_hip_qk_norm_rope_store(q, k, v, q_norm, k_norm, heads, kv_heads, head_dim, position,
                                                     theta, eps, k_cache, v_cache));
}

namespace {
citlali_hip_norm to_abi(const NormInput& n) { return citlali_hip_norm{n.delta, n.weight, n.sum_out, n.eps}; }
// weight types the grouped / fused GEMV kernels read
bool fusable(GgufTensorType t) {
    return t == GgufTensorType::Q4_K || t == GgufTensorType::Q6_K || t == GgufTensorType::F16;
}
bool launched(int st) {
    if (st == CITLALI_ERR_UNSUPPORTED) return false;
    CITLALI_HIP_CHECK(st);
    return true;
}
}  // namespace

bool launch_matvec_group(int count, const GgufTensorType* types, const uint8_t* const* weights,
                         const uint16_t* input, uint16_t* const* outputs, const int* out_features, int in_features) {
    require(count >= 1 && count <= 3, "launch_matvec_group: count must be 1, 2 or 3");
    int codes[3];
    for (int i = 0; i < count; ++i) {
        if (!fusable(types[i])) return false;
        codes[i] = static_cast<int>(types[i]);
    }
    return launched(citlali_hip_matvec_group(count, codes, weights, input, outputs, out_features, in_features));
}

bool launch_matvec_group_norm(int count, const GgufTensorType* types, const uint8_t* const* weights,
                              const uint16_t* input, const NormInput& norm, uint16_t* const* outputs,
                              const int* out_features, int in_features) {
    require(count >= 1 && count <= 3, "launch_matvec_group_norm: count must be 1, 2 or 3");
    int codes[3];
    for (int i = 0; i < count; ++i) {
        if (!fusable(types[i])) return false;
        codes[i] = static_cast<int>(types[i]);
    }
    const citlali_hip_norm n = to_abi(norm);
    return launched(citlali_hip_matvec_group_norm(count, codes, weights, input, &n, outputs, out_features,
                                                  in_features));
}

bool launch_matvec_gate_up_swiglu_norm(GgufTensorType type, const uint8_t* w_gate, const uint8_t* w_up,
                                       const uint16_t* input, const NormInput& norm, uint16_t* output,
                                       int in_features, int out_features) {
    if (!fusable(type)) return false;
    const citlali_hip_norm n = to_abi(norm);
    return launched(citlali_hip_matvec_gate_up_swiglu_norm(static_cast<int>(type), w_gate, w_up, input, &n, output,
                                                           in_features, out_features));
}

bool launch_matvec_norm(GgufTensorType type, const uint8_t* weight, const uint16_t* input, const NormInput& norm,
                        void* output, bool f32_out, int in_features, int out_features) {
    if (!fusable(type)) return false;
    const citlali_hip_norm n = to_abi(norm);
    return launched(citlali_hip_matvec_norm(static_cast<int>(type), weight, input, &n, output, f32_out ? 1 : 0,
                                            in_features, out_features));
}

bool launch_matvec_gate_up_swiglu(GgufTensorType type, const uint8_t* w_gate, const uint8_t* w_up,
                                  const uint16_t* input, uint16_t* output, int in_features, int out_features) {
    if (!fusable(type)) return false;
    return launched(citlali_hip_matvec_gate_up_swiglu(static_cast<int>(type), w_gate, w_up, input, output,
                                                      in_features, out_features));
}

void launch_argmax(const float* logits, int n, int32_t* out_index) {
    CITLALI_HIP_CHECK(citlali_hip_argmax(logits, n, out_index));
}

bool launch_qk_norm_rope_store_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                         const uint16_t* q_norm, const uint16_t* k_norm, int heads, int kv_heads,
                                         int head_dim, int position, const int32_t* position_at, int plan_length,
                                         int max_context, float theta, float eps, uint16_t* k_cache,
                                         uint16_t* v_cache, float* workspace, std::size_t workspace_bytes,
                                         uint16_t* output) {
    const int st = citlali_hip_qk_norm_rope_store_attention(q, k, v, q_norm, k_norm, heads, kv_heads, head_dim,
                                                            position, position_at, plan_length, max_context, theta,
                                                            eps, k_cache, v_cache, workspace, workspace_bytes, output);
    if (st == CITLALI_ERR_UNSUPPORTED) return false;
    CITLALI_HIP_CHECK(st);
    return true;
}

void synchronize() { CITLALI_HIP_CHECK(citlali_hip_synchronize()); }

void launch_dequant_q4k_f16(const uint8_t* blocks, uint64_t count, uint16_t* output) {
    CITLALI_HIP_CHECK(citlali_hip_dequant_q4k_f16(blocks, count, output));
}

void launch_dequant_q6k_f16(const uint8_t* blocks, uint64_t count, uint16_t* output) {
    CITLALI_HIP_CHECK(citlali_hip_dequant_q6k_f16(blocks, count, output));
}

void launch_embed_q6k_at(const uint8_t* embedding, const int32_t* token, int vocab, uint16_t* output, int hidden) {
    CITLALI_HIP_CHECK(citlali_hip_embed_q6k_at(embedding, token, vocab, output, hidden));
}

void launch_embed_at(const uint16_t* embedding, const int32_t* token, int vocab, uint16_t* output, int hidden) {
    CITLALI_HIP_CHECK(citlali_hip_embed_at(embedding, token, vocab, output, hidden));
}

void launch_qk_norm_rope_store_at(uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                                  const uint16_t* k_norm, int heads, int kv_heads, int head_dim,
                                  const int32_t* position, int max_positions, float theta, float eps,
                                  uint16_t* k_cache, uint16_t* v_cache) {
    CITLALI_HIP_CHECK(citlali_hip_qk_norm_rope_store_at(q, k, v, q_norm, k_norm, heads, kv_heads, head_dim, position,
                                                        max_positions, theta, eps, k_cache, v_cache));
}

void launch_attention_at(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         const int32_t* position, int plan_length, float* workspace, std::size_t workspace_bytes,
                         uint16_t* output, int heads, int kv_heads, int head_dim) {
    CITLALI_HIP_CHECK(citlali_hip_attention_batched(q, k_cache, v_cache, 0, position, plan_length, 1, heads, kv_heads,
                                                    head_dim, workspace, workspace_bytes, output));
}

int attention_plan_length(int length, int max_context) {
    const int n = citlali_hip_attention_plan_length(length, max_context);
    require(n > 0, "attention_plan_length: length outside [1, max_context]");
    return n;
}

std::size_t attention_workspace_bytes(int length, int heads, int kv_heads, int head_dim) {
    return citlali_hip_attention_workspace_bytes(length, 1, heads, kv_heads, head_dim);
}

void launch_argmax_advance(const float* logits, int n, int32_t* state, int32_t* tokens, int capacity) {
    CITLALI_HIP_CHECK(citlali_hip_argmax_advance(logits, n, state, tokens, capacity));
}

void* create_stream() {
    void* s = nullptr;
    CITLALI_HIP_CHECK(citlali_hip_stream_create(&s));
    return s;
}

void destroy_stream(void* stream) noexcept {
    if (stream) (void)citlali_hip_stream_destroy(stream);
}

void* current_stream() { return citlali_hip_get_stream(); }

void set_stream(void* stream) { CITLALI_HIP_CHECK(citlali_hip_set_stream(stream)); }

void graph_begin() { CITLALI_HIP_CHECK(citlali_hip_graph_begin()); }

void* graph_end() {
    void* g = nullptr;
    CITLALI_HIP_CHECK(citlali_hip_graph_end(&g));
    return g;
}

void graph_launch(void* graph) { CITLALI_HIP_CHECK(citlali_hip_graph_launch(graph)); }

void graph_destroy(void* graph) noexcept {
    if (graph) (void)citlali_hip_graph_destroy(graph);
}

}  // namespace citlali::compute
