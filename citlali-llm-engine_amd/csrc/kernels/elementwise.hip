// elementwise.hip -- the remaining kernels of one decode step
// (kernels.cu:27-124, 381-533 of the reference) and a device greedy argmax.
//
// Arithmetic follows the reference: fp16 loads widened exactly, fp32 math,
// fp16 stores rounded nearest-even.
#include "device_common.hpp"
#include "launch.hpp"
#include "citlali_hip.h"

#include <math.h>

namespace citlali::hip {
namespace {

constexpr int kBlk = 256;

__global__ void store_kv_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int position, int kv_size) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < kv_size) {
        const size_t o = (size_t)position * kv_size + i;
        kc[o] = k[i];
        vc[o] = v[i];
    }
}

// token from `token_at` (device) when not null: outside [0, vocab) -> zeros
__global__ void embed_f16_kernel(const uint16_t* __restrict__ t, int32_t token_id, const int32_t* __restrict__ token_at,
                                 int vocab, uint16_t* __restrict__ out, int hidden) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hidden) return;
    if (token_at) {
        token_id = *token_at;
        if (token_id < 0 || token_id >= vocab) {
            out[i] = 0;
            return;
        }
    }
    out[i] = t[(size_t)token_id * hidden + i];
}

__global__ void copy_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = in[i];
}

__global__ void add_inplace_kernel(uint16_t* __restrict__ t, const uint16_t* __restrict__ d, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) t[i] = f2h_rne(h2f(t[i]) + h2f(d[i]));
}

// sum of squares over one block, result in every thread
__device__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
    const int nw = blockDim.x / kWave;
    for (int w = 0; w < nw; ++w) s += red[w];
    __syncthreads();
    return s;
}

// one block per head (rms_norm_heads: `heads` vectors, weight shared by all
// heads)
__global__ void rms_norm_kernel(const uint16_t* __restrict__ in, const uint16_t* __restrict__ w,
                                uint16_t* __restrict__ out, int n, float eps) {
    __shared__ float red[16];
    const size_t base = (size_t)blockIdx.x * n;
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = h2f(in[base + i]);
        s += v * v;
    }
    s = block_sum(s, red);
    const float inv = rsqrtf(s / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[base + i] = f2h_rne(h2f(in[base + i]) * inv * h2f(w[i]));
}

// RMSNorm of one vector (launch_rms_norm, kernels.cu:67-92) in the run order
// of device_common.hpp shared with add_rms_norm_kernel and the GEMV input
// prologue, so the three agree bit for bit.
__global__ __launch_bounds__(kNormThreads) void rms_norm_vec_kernel(const uint16_t* __restrict__ in,
                                                                    const uint16_t* __restrict__ w,
                                                                    uint16_t* __restrict__ out, int n, float eps) {
    __shared__ float red[4];
    float s = 0.f;
    for (int r = threadIdx.x; r * 8 < n; r += kNormThreads)
        for (int j = 0; j < 8; ++j) {
            const int i = r * 8 + j;
            if (i < n) {
                const float v = h2f(in[i]);
                s += v * v;
            }
        }
    s = norm_block_sum(s, red);
    const float inv = rsqrtf(s / (float)n + eps);
    for (int r = threadIdx.x; r * 8 < n; r += kNormThreads)
        for (int j = 0; j < 8; ++j) {
            const int i = r * 8 + j;
            if (i < n) out[i] = f2h_rne(h2f(in[i]) * inv * h2f(w[i]));
        }
}

// Residual add then RMSNorm of the sum, one launch for the reference's
// launch_add_inplace + launch_rms_norm pair (qwen_model.cpp:340-341, 372 and
// the next layer's 306 or the final norm at 385): x = fp16(x + d) is stored,
// then norm = fp16(x * rsqrt(mean(x^2) + eps) * w) over the stored values.
// One 256-thread block in the order of device_common.hpp's run helpers --
// the order the GEMVs' norm prologue uses, so a GEMV fed by this kernel and
// the GEMV with the prologue give the same results bit for bit.
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(uint16_t* __restrict__ x,
                                                                    const uint16_t* __restrict__ d,
                                                                    const uint16_t* __restrict__ w,
                                                                    uint16_t* __restrict__ out, int n, float eps) {
    __shared__ float red[4];
    float s = 0.f;
    for (int r = threadIdx.x; r * 8 < n; r += kNormThreads) {
        for (int j = 0; j < 8; ++j) {
            const int i = r * 8 + j;
            if (i < n) {
                const uint16_t xi = f2h_rne(h2f(x[i]) + h2f(d[i]));
                x[i] = xi;
                const float v = h2f(xi);
                s += v * v;
            }
        }
    }
    s = norm_block_sum(s, red);
    const float inv = rsqrtf(s / (float)n + eps);
    for (int r = threadIdx.x; r * 8 < n; r += kNormThreads)
        for (int j = 0; j < 8; ++j) {
            const int i = r * 8 + j;
            if (i < n) out[i] = f2h_rne(h2f(x[i]) * inv * h2f(w[i]));
        }
}

// Per-head RMSNorm of q and k (when their weights are given), NeoX RoPE of
// both, and the store of this position's k and v rows into the caches: the
// reference's launch_rms_norm_heads x2, launch_rope x2 and launch_store_kv
// (qwen_model.cpp:326-336) in one launch.  Block h < heads is query head h
// (rewritten in place); block heads + j is kv head j (k roped into k_cache,
// v copied into v_cache).  Each stage rounds to fp16 where the separate
// kernels store, with the same per-head 128-thread reduction, so the
// results equal the separate launches bit for bit.
// The position comes from `position_at` (device memory) when that is not
// null; a position there outside [0, max_positions) writes nothing to the
// caches (the host validates the scalar form).
__global__ void qk_norm_rope_store_kernel(uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                          const uint16_t* __restrict__ v, const uint16_t* __restrict__ qw,
                                          const uint16_t* __restrict__ kw, int heads, int head_dim, int position,
                                          const int32_t* __restrict__ position_at, int max_positions, float theta,
                                          float eps, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                                          int kv_size) {
    __shared__ float red[16];
    __shared__ uint16_t vals[256];
    const bool is_q = (int)blockIdx.x < heads;
    if (position_at) {
        position = *position_at;
        if (!is_q && (position < 0 || position >= max_positions)) return;   // whole block: no barrier skipped
    }
    const int head = is_q ? blockIdx.x : blockIdx.x - heads;
    const uint16_t* src = is_q ? q + (size_t)head * head_dim : k + (size_t)head * head_dim;
    const uint16_t* w = is_q ? qw : kw;
    const int i = threadIdx.x;   // blockDim.x == 128 >= head_dim
    uint16_t xi = i < head_dim ? src[i] : (uint16_t)0;
    if (w != nullptr) {
        const float xv = h2f(xi);
        const float ss = block_sum(i < head_dim ? xv * xv : 0.f, red);
        const float inv = rsqrtf(ss / (float)head_dim + eps);
        if (i < head_dim) xi = f2h_rne(xv * inv * h2f(w[i]));
    }
    if (i < head_dim) vals[i] = xi;
    __syncthreads();
    const int half = head_dim / 2;
    uint16_t* dst = is_q ? q + (size_t)head * head_dim
                         : k_cache + (size_t)position * kv_size + (size_t)head * head_dim;
    if (i < half) {
        uint16_t y0, y1;
        rope_pair(h2f(vals[i]), h2f(vals[half + i]), i, head_dim, position, theta, y0, y1);
        dst[i] = y0;
        dst[half + i] = y1;
    }
    if (!is_q && i < head_dim)
        v_cache[(size_t)position * kv_size + (size_t)head * head_dim + i] = v[(size_t)head * head_dim + i];
}

// NeoX pairs (i, i + hd/2), angle = position * theta^(-2i/hd) (kernels.cu:485-521)
__global__ void rope_kernel(uint16_t* __restrict__ data, int head_dim, int position, float theta) {
    const int head = blockIdx.x, i = threadIdx.x, half = head_dim / 2;
    if (i >= half) return;
    const size_t base = (size_t)head * head_dim;
    uint16_t y0, y1;
    rope_pair(h2f(data[base + i]), h2f(data[base + half + i]), i, head_dim, position, theta, y0, y1);
    data[base + i] = y0;
    data[base + half + i] = y1;
}

__global__ void swiglu_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                              uint16_t* __restrict__ out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float gv = h2f(g[i]);
        out[i] = f2h_rne(gv / (1.0f + expf(-gv)) * h2f(u[i]));
    }
}

// fp16 weights [N][K] (the DequantizeToFp16 path) for K not a multiple of
// 256: one wave per row, 128-bit loads when K is a multiple of 8, fp32
// accumulation.
template <bool kF32>
__global__ __launch_bounds__(kBlk) void matvec_f16_kernel(const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ x, void* __restrict__ y,
                                                          int K, int N) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * (kBlk / kWave) + threadIdx.x / kWave;
    if (row >= N) return;
    const uint16_t* r = w + (size_t)row * K;
    float a = 0.f;
    if ((K & 7) == 0) {
        for (int k = lane * 8; k < K; k += kWave * 8) {
            const u32x4 wv = *reinterpret_cast<const u32x4*>(r + k);
            const u32x4 xv = *reinterpret_cast<const u32x4*>(x + k);
            a = dot2(wv.x, xv.x, a);
            a = dot2(wv.y, xv.y, a);
            a = dot2(wv.z, xv.z, a);
            a = dot2(wv.w, xv.w, a);
        }
    } else {
        for (int k = lane; k < K; k += kWave) a = fmaf(h2f(r[k]), h2f(x[k]), a);
    }
    a = wave_sum(a);
    if (lane == 0) {
        if constexpr (kF32) static_cast<float*>(y)[row] = a;
        else static_cast<uint16_t*>(y)[row] = f2h_rne(a);
    }
}

// Greedy argmax with the host rule of qwen_model.cpp:455-463: the first
// (lowest index) strictly greatest finite value wins; all non-finite -> 0.
// Two launches: blocks reduce contiguous ranges to a partial, one block
// reduces the partials.  A candidate is one 64-bit key, (order-preserving
// bits of the value) << 32 | ~index, so the largest key is the largest value
// and, among equal values, the lowest index; -0.0 counts as +0.0, as the
// host's `>` does.  0 means "no finite value".
constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxMaxBlocks = 1024;
__device__ uint64_t g_argmax_partial[kArgmaxMaxBlocks];   // per device; concurrent argmax calls would race

__device__ __forceinline__ uint64_t argmax_key(float v, int i) {
    if (!isfinite(v)) return 0ull;
    uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)~(uint32_t)i;
}

__device__ __forceinline__ uint64_t block_max_u64(uint64_t k, uint64_t* red) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const uint64_t o = __shfl_xor(k, off, kWave);
        k = o > k ? o : k;
    }
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == 0) red[wave] = k;
    __syncthreads();
    uint64_t m = 0;
    for (int w = 0; w < (int)(blockDim.x / kWave); ++w) m = red[w] > m ? red[w] : m;
    return m;
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial_kernel(const float* __restrict__ logits, int n,
                                                                         int per_block) {
    __shared__ uint64_t red[kArgmaxThreads / kWave];
    const int b0 = blockIdx.x * per_block, b1 = min(n, b0 + per_block);
    uint64_t k = 0;
    for (int i = b0 + (int)threadIdx.x; i < b1; i += kArgmaxThreads) {
        const uint64_t c = argmax_key(logits[i], i);
        k = c > k ? c : k;
    }
    const uint64_t m = block_max_u64(k, red);
    if (threadIdx.x == 0) g_argmax_partial[blockIdx.x] = m;
}

// With `state` (device int32 {token, position, step, 0}) the pick also
// becomes the next step's input: tokens[step] = pick (while step <
// capacity), token = pick, position += 1, step += 1.
__global__ __launch_bounds__(kArgmaxThreads) void argmax_final_kernel(int parts, int32_t* __restrict__ out,
                                                                      int32_t* __restrict__ state,
                                                                      int32_t* __restrict__ tokens, int capacity) {
    __shared__ uint64_t red[kArgmaxThreads / kWave];
    // the position and step are read with the partials, not after the
    // reduction
    const bool lead = state && threadIdx.x == 0;
    const int32_t position = lead ? state[1] : 0, step = lead ? state[2] : 0;
    uint64_t k = 0;
    for (int i = threadIdx.x; i < parts; i += kArgmaxThreads) k = g_argmax_partial[i] > k ? g_argmax_partial[i] : k;
    const uint64_t m = block_max_u64(k, red);
    if (threadIdx.x == 0) {
        const int32_t pick = m == 0 ? 0 : (int32_t)~(uint32_t)(m & 0xffffffffu);
        if (out) out[0] = pick;
        if (state) {
            if (step >= 0 && step < capacity) tokens[step] = pick;
            state[0] = pick;
            state[1] = position + 1;
            state[2] = step + 1;
        }
    }
}

__global__ void fill_zero_kernel(uint32_t* __restrict__ p, size_t nwords) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nwords; i += stride) p[i] = 0u;
}

__global__ void fill_zero_bytes_kernel(uint8_t* __restrict__ p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Streaming read of a large buffer (the achievable HBM read ceiling): each
// workgroup reads one contiguous slab, four 16-byte nontemporal loads in
// flight per lane, so every load instruction covers whole cache lines (the
// fastest of the grid-stride / slab and plain / nontemporal patterns, about
// 7.1 TB/s on a 2 GiB buffer); the last workgroup also reads the remainder.
// The xor of the data is written only if it equals a value the caller never
// stores, so the loads cannot be dropped.
__global__ __launch_bounds__(kBlk) void stream_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                           uint32_t* __restrict__ sink) {
    constexpr int kU = 4;
    const size_t per = n16 / gridDim.x;
    const u32x4* q = p + (size_t)blockIdx.x * per;
    u32x4 a[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) a[u] = u32x4{0u, 0u, 0u, 0u};
    size_t i = threadIdx.x;
    for (; i + (kU - 1) * kBlk < per; i += kU * kBlk) {
#pragma unroll
        for (int u = 0; u < kU; ++u) a[u] ^= __builtin_nontemporal_load(q + i + u * kBlk);
    }
    for (; i < per; i += kBlk) a[0] ^= __builtin_nontemporal_load(q + i);
    if (blockIdx.x == gridDim.x - 1)
        for (size_t j = per * gridDim.x + threadIdx.x; j < n16; j += kBlk) a[0] ^= p[j];
#pragma unroll
    for (int u = 1; u < kU; ++u) a[0] ^= a[u];
    const uint32_t v = a[0].x ^ a[0].y ^ a[0].z ^ a[0].w;
    if (v == 0x9e3779b9u) sink[0] = v;
}

inline dim3 grid_for(int n) { return dim3((unsigned)((n + kBlk - 1) / kBlk)); }

}  // namespace

hipError_t launch_store_kv(const uint16_t* k, const uint16_t* v, uint16_t* kc, uint16_t* vc, int position,
                           int kv_size, hipStream_t s) {
    launch_kernel(store_kv_kernel, grid_for(kv_size), dim3(kBlk), 0, s, k, v, kc, vc, position, kv_size);
    return hipGetLastError();
}

hipError_t launch_embed_f16(const uint16_t* t, int32_t token_id, const int32_t* token_at, int vocab, uint16_t* out,
                            int hidden, hipStream_t s) {
    launch_kernel(embed_f16_kernel, grid_for(hidden), dim3(kBlk), 0, s, t, token_id, token_at, vocab, out, hidden);
    return hipGetLastError();
}

hipError_t launch_copy(const uint16_t* in, uint16_t* out, int n, hipStream_t s) {
    launch_kernel(copy_kernel, grid_for(n), dim3(kBlk), 0, s, in, out, n);
    return hipGetLastError();
}

hipError_t launch_add_inplace(uint16_t* t, const uint16_t* d, int n, hipStream_t s) {
    launch_kernel(add_inplace_kernel, grid_for(n), dim3(kBlk), 0, s, t, d, n);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const uint16_t* in, const uint16_t* w, uint16_t* out, int n, float eps, hipStream_t s) {
    launch_kernel(rms_norm_vec_kernel, dim3(1), dim3(kNormThreads), 0, s, in, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_rms_norm_heads(const uint16_t* in, const uint16_t* w, uint16_t* out, int heads, int head_dim,
                                 float eps, hipStream_t s) {
    launch_kernel(rms_norm_kernel, dim3(heads), dim3(kWave * 2), 0, s, in, w, out, head_dim, eps);
    return hipGetLastError();
}

hipError_t launch_add_rms_norm(uint16_t* x, const uint16_t* d, const uint16_t* w, uint16_t* out, int n, float eps,
                               hipStream_t s) {
    launch_kernel(add_rms_norm_kernel, dim3(1), dim3(kNormThreads), 0, s, x, d, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_qk_norm_rope_store(uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* qw,
                                     const uint16_t* kw, int heads, int kv_heads, int head_dim, int position,
                                     const int32_t* position_at, int max_positions, float theta, float eps,
                                     uint16_t* k_cache, uint16_t* v_cache, hipStream_t s) {
    launch_kernel(qk_norm_rope_store_kernel, dim3(heads + kv_heads), dim3(kWave * 2), 0, s, q, k, v, qw, kw, heads,
                  head_dim, position, position_at, max_positions, theta, eps, k_cache, v_cache, kv_heads * head_dim);
    return hipGetLastError();
}

hipError_t launch_rope(uint16_t* data, int heads, int head_dim, int position, float theta, hipStream_t s) {
    const int threads = ((head_dim / 2 + kWave - 1) / kWave) * kWave;
    launch_kernel(rope_kernel, dim3(heads), dim3(threads), 0, s, data, head_dim, position, theta);
    return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t* g, const uint16_t* u, uint16_t* out, int n, hipStream_t s) {
    launch_kernel(swiglu_kernel, grid_for(n), dim3(kBlk), 0, s, g, u, out, n);
    return hipGetLastError();
}

hipError_t launch_matvec_f16(const uint16_t* w, const uint16_t* x, void* y, bool f32_out, int K, int N,
                             hipStream_t s) {
    // whole 256-value blocks: the streaming GEMV kernels (the fused fp16
    // launches use the same ones, so their results are these bits)
    if (K % 256 == 0 && K <= CITLALI_MAX_IN_FEATURES) return launch_matvec_f16_blocks(w, x, y, f32_out, K, N, s);
    const dim3 g((unsigned)((N + (kBlk / kWave) - 1) / (kBlk / kWave)));
    if (f32_out) launch_kernel(matvec_f16_kernel<true>, g, dim3(kBlk), 0, s, w, x, y, K, N);
    else launch_kernel(matvec_f16_kernel<false>, g, dim3(kBlk), 0, s, w, x, y, K, N);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int n, int32_t* out_index, int32_t* state, int32_t* tokens,
                         int capacity, hipStream_t s) {
    // about 4 values per thread, at most kArgmaxMaxBlocks partials
    int parts = (n + 4 * kArgmaxThreads - 1) / (4 * kArgmaxThreads);
    if (parts > kArgmaxMaxBlocks) parts = kArgmaxMaxBlocks;
    const int per_block = (n + parts - 1) / parts;
    parts = (n + per_block - 1) / per_block;
    launch_kernel_in_call(false, argmax_partial_kernel, dim3(parts), dim3(kArgmaxThreads), 0, s, logits, n, per_block);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_kernel(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, s, parts, out_index, state, tokens,
                  capacity);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* sink, hipStream_t s) {
    int dev = 0, cus = 256;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const size_t n16 = bytes / 16;
    launch_kernel(stream_read_kernel, dim3((unsigned)(cus * 4)), dim3(kBlk), 0, s,
                       static_cast<const u32x4*>(buf), n16, sink);
    return hipGetLastError();
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s) {
    if (bytes == 0) return hipSuccess;
    if (((uintptr_t)p & 3u) == 0 && (bytes & 3u) == 0) {
        const size_t words = bytes / 4;
        size_t blocks = (words + kBlk - 1) / kBlk;
        if (blocks > 65536) blocks = 65536;
        launch_kernel(fill_zero_kernel, dim3((unsigned)blocks), dim3(kBlk), 0, s, (uint32_t*)p, words);
    } else {
        size_t blocks = (bytes + kBlk - 1) / kBlk;
        launch_kernel(fill_zero_bytes_kernel, dim3((unsigned)blocks), dim3(kBlk), 0, s, (uint8_t*)p, bytes);
    }
    return hipGetLastError();
}

}  // namespace citlali::hip
