// launch.hpp -- internal launchers of the gfx950 kernels, called by the
// C-ABI layer (csrc/abi/citlali_hip.hip) after it has validated arguments.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

namespace citlali::hip {

// ---- kernel timing (citlali_hip_set_kernel_timing) ----
// While armed on a thread, the first kernel that thread launches records
// `start` when it begins and the last kernel of each call records `stop`
// when it ends (hipExtLaunchKernel stamps the events from the dispatch
// itself), so the elapsed time is the kernels' own time, without the
// queueing gap an event recorded on the stream would add.
// Per-dispatch mode (citlali_hip_set_dispatch_timing): while `starts` is not
// empty, the i-th kernel launched (i < starts.size()) records starts[i] when
// it begins and stops[i] when it ends; `used` counts every kernel launched
// while armed, stamped or not.
struct KernelTiming {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    std::vector<hipEvent_t> starts, stops;
    int used = 0;
};
KernelTiming& kernel_timing();   // thread-local state, defined by the ABI unit

// Every launch of the library goes through here; `last` is false for a
// kernel that another kernel of the same call follows.
template <typename Kernel, typename... Args>
inline void launch_kernel_in_call(bool last, Kernel kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                                  Args... args) {
    KernelTiming& t = kernel_timing();
    if (!t.starts.empty()) {
        const size_t i = (size_t)t.used++;
        if (i < t.starts.size()) {
            hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, t.starts[i], t.stops[i], 0u, args...);
        } else {
            hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
        }
        return;
    }
    if (t.start == nullptr && (t.stop == nullptr || !last)) {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
        return;
    }
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, t.start, last ? t.stop : nullptr, 0u,
                          args...);
    t.start = nullptr;
}

template <typename Kernel, typename... Args>
inline void launch_kernel(Kernel kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, Args... args) {
    launch_kernel_in_call(true, kernel, grid, block, lds, stream, args...);
}

// ---- fused dequant GEMV (matvec_kquant.hip) ----
// kind: 4 = Q4_K, 6 = Q6_K, 1 = fp16 weights
size_t matvec_lds_bytes(int kind, int K);
// in_features the streaming kernels cover: 1024, 2048, 2560, 3072, 4096,
// 5120, 6144, 8192, 9728, 12288, 16384 (the grouped GEMV and the input
// prologue take these), and with norm = false also 17408 and 25600 (plain
// K-quant GEMVs)
bool matvec_fused_length(int K, bool norm);
// in_features of the gate/up + SwiGLU launch: 1024, 2048, 2560, 3072, 4096,
// 5120, 8192
bool matvec_gate_up_length(int K);
// fp16 weights [N][K], K a multiple of 256 up to CITLALI_MAX_IN_FEATURES,
// through the streaming kernels of the K-quant GEMVs
hipError_t launch_matvec_f16_blocks(const uint16_t* w, const uint16_t* x, void* y, bool f32_out, int K, int N,
                                    hipStream_t s);
hipError_t launch_matvec_q4k(const uint8_t* w, const uint16_t* x, void* y, bool f32_out, int K, int N,
                             hipStream_t s);
hipError_t launch_matvec_q6k(const uint8_t* w, const uint16_t* x, void* y, bool f32_out, int K, int N,
                             hipStream_t s);

// ---- decode attention (attention.hip) ----
// The step's q/k head RMSNorm + RoPE and KV store done inside the attention
// launch (head_dim 128, GQA group 2..8): k and v of this step before the
// norm ([nseq][kv_heads][128]), the norm weights (null: no norm), writable
// views of the caches.  Attention then reads q as it comes from the q GEMV.
struct QkPrep {
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    uint16_t* k_cache;
    uint16_t* v_cache;
    float theta, eps;
};
struct AttnArgs {
    const uint16_t* q;         // [nseq][heads][head_dim]
    const uint16_t* k_cache;   // sequence s at k_cache + s*seq_stride: [pos][kv_heads][head_dim]
    const uint16_t* v_cache;
    long long seq_stride;      // elements
    const int32_t* positions;  // device [nseq] or null (then `position`)
    int position;
    int max_len;               // positions past max_len - 1 are ignored (the plan's bound)
    int nseq, heads, kv_heads, head_dim;
    float* workspace;          // chunk partials, attention_workspace_bytes()
    uint16_t* out;             // [nseq][heads][head_dim]
    const QkPrep* prep;        // null: q already normed and roped, the step's k/v already stored
};
struct AttnPlan {
    int gp;        // padded GQA group (1, 2, 4, 8)
    int chunk;     // positions per workgroup
    int n_splits;  // chunks of the longest sequence
    int depth;     // K/V tiles in flight per wave (1 or 2; the matrix-core kernel takes 1)
    bool rows;     // matrix-core kernel: whole-row nontemporal tile loads through LDS
};
bool attention_supported(int head_dim, int group);
// The length a decode step's attention is planned for: the smallest power
// of two >= max(length, 256), at most max_context.
int attention_plan_length(int length, int max_context);
AttnPlan plan_attention(int max_len, int nseq, int kv_heads, int heads, int head_dim, int target_blocks);
size_t attention_workspace_bytes(const AttnPlan& p, int nseq, int heads, int head_dim);
// Bytes that hold the partials of the plan for every length in [1, max_len].
size_t attention_workspace_bound(int max_len, int nseq, int kv_heads, int heads, int head_dim, int target_blocks);
hipError_t launch_attention(const AttnArgs& a, const AttnPlan& p, hipStream_t s);

// ---- embedding / dequant (dequant.hip) ----
// token_at (device, may be null) replaces token_id; out of [0, vocab) -> zeros
hipError_t launch_embed_q6k(const uint8_t* table, int32_t token_id, const int32_t* token_at, int vocab,
                            uint16_t* out, int hidden, hipStream_t s);
hipError_t launch_dequant_q4k_f16(const uint8_t* w, uint64_t count, uint16_t* out, hipStream_t s);
hipError_t launch_dequant_q6k_f16(const uint8_t* w, uint64_t count, uint16_t* out, hipStream_t s);

// ---- the rest of the decode step (elementwise.hip) ----
hipError_t launch_store_kv(const uint16_t* k, const uint16_t* v, uint16_t* kc, uint16_t* vc, int position,
                           int kv_size, hipStream_t s);
hipError_t launch_embed_f16(const uint16_t* table, int32_t token_id, const int32_t* token_at, int vocab,
                            uint16_t* out, int hidden, hipStream_t s);
hipError_t launch_copy(const uint16_t* in, uint16_t* out, int n, hipStream_t s);
hipError_t launch_add_inplace(uint16_t* t, const uint16_t* d, int n, hipStream_t s);
hipError_t launch_rms_norm(const uint16_t* in, const uint16_t* w, uint16_t* out, int n, float eps,
                           hipStream_t s);
hipError_t launch_rms_norm_heads(const uint16_t* in, const uint16_t* w, uint16_t* out, int heads, int head_dim,
                                 float eps, hipStream_t s);
hipError_t launch_rope(uint16_t* data, int heads, int head_dim, int position, float theta, hipStream_t s);
hipError_t launch_swiglu(const uint16_t* g, const uint16_t* u, uint16_t* out, int n, hipStream_t s);
hipError_t launch_matvec_f16(const uint16_t* w, const uint16_t* x, void* y, bool f32_out, int K, int N,
                             hipStream_t s);
// out_index and/or the decode state {token, position, step, 0} (device)
hipError_t launch_argmax(const float* logits, int n, int32_t* out_index, int32_t* state, int32_t* tokens,
                         int capacity, hipStream_t s);
// fused forward_token steps (no reference counterpart; same results as the
// separate launches)
hipError_t launch_add_rms_norm(uint16_t* x, const uint16_t* d, const uint16_t* w, uint16_t* out, int n, float eps,
                               hipStream_t s);
hipError_t launch_qk_norm_rope_store(uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* qw,
                                     const uint16_t* kw, int heads, int kv_heads, int head_dim, int position,
                                     const int32_t* position_at, int max_positions, float theta, float eps,
                                     uint16_t* k_cache, uint16_t* v_cache, hipStream_t s);
// GEMV input prologue (residual add + RMSNorm): the GEMV reads
// fp16(xs * rsqrt(mean(xs^2) + eps) * w) with xs = fp16(x + d) (xs = x when
// d is null); workgroup 0 stores xs to xs_out when that is not null.  Equal
// bit for bit to launch_add_rms_norm followed by the plain GEMV.
struct NormIn {
    const uint16_t* d;
    const uint16_t* w;
    uint16_t* xs_out;
    float eps;
};
hipError_t launch_matvec_group(int count, const int* kinds, const uint8_t* const* w, const uint16_t* x,
                               uint16_t* const* y, const int* n, int K, const NormIn* norm, hipStream_t s);
hipError_t launch_matvec_gate_up_swiglu(int kind, const uint8_t* wg, const uint8_t* wu, const uint16_t* x,
                                        uint16_t* act, int K, int N, const NormIn* norm, hipStream_t s);
// kind 4 / 6 / 1 GEMV with the input prologue; K 1024, 2048, 3072 or a
// multiple of 4096 up to 16384
hipError_t launch_matvec_norm(int kind, const uint8_t* w, const uint16_t* x, const NormIn& norm, void* y,
                              bool f32_out, int K, int N, hipStream_t s);
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s);
hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* sink, hipStream_t s);

}  // namespace citlali::hip
