// citlali/compute/hip/kernels.h -- the launchers the model code calls.
//
// Same signatures and meaning as the reference's compute layer
// (include/citlali/compute/cuda/kernels.h:8-61), implemented over the C ABI
// of libcitlali_hip.so (gfx950 kernels).  Launches are asynchronous on the
// library stream; failures throw citlali::Error.  `cuda_zero` is named
// `device_zero` here.
#pragma once

#include <cstddef>
#include <cstdint>

namespace citlali::compute {

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
// Greedy pick on the device (no reference counterpart: the reference copies
// the logits to the host, qwen_model.cpp:448-465): the first largest finite
// value of logits[0..n) is written to *out_index (0 when none is finite).
void launch_argmax(const float* logits, int n, int32_t* out_index);
// Waits for every launch queued on the library stream.
void synchronize();

}  // namespace citlali::compute
