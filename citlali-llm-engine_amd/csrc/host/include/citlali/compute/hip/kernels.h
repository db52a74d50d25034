// citlali/compute/hip/kernels.h -- the launchers the model code calls.
//
// Same signatures and meaning as the reference's compute layer
// (include/citlali/compute/cuda/kernels.h:8-61), implemented over the C ABI
// of libcitlali_hip.so (gfx950 kernels).  Launches are asynchronous on the
// library stream; failures throw citlali::Error.  `cuda_zero` keeps its
// reference name (kernels.h:8); `device_zero` is the same call.
#pragma once

#include "citlali/compute/common/dtype.h"

#include <cstddef>
#include <cstdint>

namespace citlali::compute {

void cuda_zero(void* data, std::size_t bytes);   // kernels.h:8, kernels.cu:655-657
void device_zero(void* data, std::size_t bytes);
void launch_embed(const uint16_t* embedding, int32_t token_id, uint16_t* out, int hidden);
void launch_copy(const uint16_t* input, uint16_t* output, int n);
void launch_add_inplace(uint16_t* target, const uint16_t* delta, int n);
void launch_add_bias_inplace(uint16_t* target, const uint16_t* bias, int n);
void launch_rms_norm(const uint16_t* input, const uint16_t* weight, uint16_t* output, int n, float eps);
void launch_rms_norm_heads(const uint16_t* input, const uint16_t* weight, uint16_t* output, int heads,
                           int head_dim, float eps);
void launch_matvec_fp16(const uint16_t* weight, const uint16_t* input, uint16_t* output, int in_features,
                        int out_features);
void launch_matvec_fp16_to_float(const uint16_t* weight, const uint16_t* input, float* output, int in_features,
                                 int out_features);
void launch_matvec_q4k(const uint8_t* weight, const uint16_t* input, uint16_t* output, int in_features,
                       int out_features);
void launch_matvec_q6k(const uint8_t* weight, const uint16_t* input, uint16_t* output, int in_features,
                       int out_features);
void launch_matvec_q6k_to_float(const uint8_t* weight, const uint16_t* input, float* output, int in_features,
                                int out_features);
void launch_embed_q6k(const uint8_t* embedding, int32_t token_id, uint16_t* output, int hidden);
void launch_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* output, int n);
void launch_rope(uint16_t* data, int heads, int head_dim, int position, float theta);
void launch_store_kv(const uint16_t* k, const uint16_t* v, uint16_t* k_cache, uint16_t* v_cache, int position,
                     int kv_size);
// `scores` (heads * max_context floats, may be null) serves as the split-KV
// workspace when large enough; it does not receive the raw scores.
void launch_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* scores,
                      uint16_t* output, int position, int max_context, int heads, int kv_heads, int head_dim);
// Fused forward_token steps (no reference counterpart): each gives the
// results of the launches it names bit for bit, in one launch.
// launch_add_inplace(x, delta) then launch_rms_norm(x, weight, output).
void launch_add_rms_norm(uint16_t* x, const uint16_t* delta, const uint16_t* weight, uint16_t* output, int n,
                         float eps);
// launch_rms_norm_heads on q and k (skipped for a null weight), launch_rope
// on both, launch_store_kv(k, v) into the caches at `position`.
void launch_qk_norm_rope_store(uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                               const uint16_t* k_norm, int heads, int kv_heads, int head_dim, int position,
                               float theta, float eps, uint16_t* k_cache, uint16_t* v_cache);
// launch_matvec_q4k / _q6k (or launch_matvec_fp16, type F16, the weight
// pointer to its fp16 rows) for `count` (1..3) weights that read the same
// input (attn_q, attn_k, attn_v); returns false, launching nothing, when a
// type is not Q4_K/Q6_K/F16, F16 is mixed with quantized types, or no
// grouped kernel covers in_features.
bool launch_matvec_group(int count, const GgufTensorType* types, const uint8_t* const* weights,
                         const uint16_t* input, uint16_t* const* outputs, const int* out_features, int in_features);
// GEMVs whose input is the residual add + RMSNorm of `input` (see
// citlali_hip_norm): the input fp16(s * rsqrt(mean(s^2) + eps) * weight),
// s = fp16(input + delta) (s = input without delta), is formed inside each
// launch, and sum_out (may be null) receives s.  The same results as
// launch_add_rms_norm / launch_rms_norm followed by the GEMV, bit for bit.
// Each returns false, launching nothing, when no kernel covers the shape or
// type.
struct NormInput {
    const uint16_t* delta;
    const uint16_t* weight;
    uint16_t* sum_out;
    float eps;
};
bool launch_matvec_group_norm(int count, const GgufTensorType* types, const uint8_t* const* weights,
                              const uint16_t* input, const NormInput& norm, uint16_t* const* outputs,
                              const int* out_features, int in_features);
bool launch_matvec_gate_up_swiglu_norm(GgufTensorType type, const uint8_t* w_gate, const uint8_t* w_up,
                                       const uint16_t* input, const NormInput& norm, uint16_t* output,
                                       int in_features, int out_features);
bool launch_matvec_norm(GgufTensorType type, const uint8_t* weight, const uint16_t* input, const NormInput& norm,
                        void* output, bool f32_out, int in_features, int out_features);
// The ffn_gate and ffn_up GEMVs (both of `type`: Q4_K, Q6_K or F16) then
// launch_swiglu; returns
// false, launching nothing, when no fused kernel covers the shape.
bool launch_matvec_gate_up_swiglu(GgufTensorType type, const uint8_t* w_gate, const uint8_t* w_up,
                                  const uint16_t* input, uint16_t* output, int in_features, int out_features);
// Greedy pick on the device (no reference counterpart: the reference copies
// the logits to the host, qwen_model.cpp:448-465): the first largest finite
// value of logits[0..n) is written to *out_index (0 when none is finite).
void launch_argmax(const float* logits, int n, int32_t* out_index);
// launch_qk_norm_rope_store(_at) followed by launch_attention(_at) in one
// launch, the same results bit for bit (q is only read); position_at (device)
// replaces `position` when not null, with plan_length the bucket.  Returns
// false, launching nothing, when no fused kernel covers the shape (head_dim
// 128 with 2..8 query heads per kv head).
bool launch_qk_norm_rope_store_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                         const uint16_t* q_norm, const uint16_t* k_norm, int heads, int kv_heads,
                                         int head_dim, int position, const int32_t* position_at, int plan_length,
                                         int max_context, float theta, float eps, uint16_t* k_cache,
                                         uint16_t* v_cache, float* workspace, std::size_t workspace_bytes,
                                         uint16_t* output);
// Waits for every launch queued on the library stream.
void synchronize();
// Load-time dequantisation on the device (no reference launcher: the
// reference dequantises on the host, weight_loader.cpp:147-323): `count`
// values of raw Q4_K / Q6_K blocks to fp16 with the host rounding rule, the
// same bits as the host routines.
void launch_dequant_q4k_f16(const uint8_t* blocks, uint64_t count, uint16_t* output);
void launch_dequant_q6k_f16(const uint8_t* blocks, uint64_t count, uint16_t* output);

// ---- replayable decode steps (no reference counterpart) -------------------
// The same launches with the token / position read from device memory
// (decode state int32 {token, position, step, 0}), so one decode step can be
// captured in a HIP graph and replayed per token; each gives the result of
// its scalar form at the values it reads.
void launch_embed_q6k_at(const uint8_t* embedding, const int32_t* token, int vocab, uint16_t* output, int hidden);
void launch_embed_at(const uint16_t* embedding, const int32_t* token, int vocab, uint16_t* output, int hidden);
void launch_qk_norm_rope_store_at(uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                                  const uint16_t* k_norm, int heads, int kv_heads, int head_dim,
                                  const int32_t* position, int max_positions, float theta, float eps,
                                  uint16_t* k_cache, uint16_t* v_cache);
// launch_attention at the position in device memory, for every position p
// with attention_plan_length(p + 1, max_context) == plan_length.
void launch_attention_at(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         const int32_t* position, int plan_length, float* workspace, std::size_t workspace_bytes,
                         uint16_t* output, int heads, int kv_heads, int head_dim);
int attention_plan_length(int length, int max_context);
// Bytes of split partials one sequence's attention planned for `length` uses.
std::size_t attention_workspace_bytes(int length, int heads, int kv_heads, int head_dim);
// launch_argmax, then tokens[step] = pick, token = pick, position += 1, step += 1
void launch_argmax_advance(const float* logits, int n, int32_t* state, int32_t* tokens, int capacity);

// Library stream and graphs (see citlali_hip_graph_begin).
void* create_stream();
void destroy_stream(void* stream) noexcept;
void* current_stream();
void set_stream(void* stream);
void graph_begin();
void* graph_end();   // ends the capture; throws when it failed
void graph_launch(void* graph);
void graph_destroy(void* graph) noexcept;

}  // namespace citlali::compute
