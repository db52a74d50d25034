// dequant.hip -- Q6_K embedding gather and whole-tensor Q4_K / Q6_K -> fp16.
//
// Values are the exact fp32 dequantised weights of kernels.cu:134-186
// (== weight_loader.cpp:147-323 before rounding).  The two entry points round
// them the way their reference counterparts do, and the reference is not
// consistent on exact ties:
//  * embed_q6k follows the reference kernel (kernels.cu:340-378), whose
//    store_half is __float2half: nearest-even.
//  * the whole-tensor dequant follows the host loader (dequant_q4_k /
//    dequant_q6_k with float_to_half_bits, dtype.cpp:136-176): nearest, ties
//    away from zero, so its output equals the host routines bit for bit.
#include "device_common.hpp"
#include "launch.hpp"

namespace citlali::hip {
namespace {

__device__ __forceinline__ float blk_half(const uint8_t* p) {
    return h2f((uint16_t)(p[0] | (p[1] << 8)));
}

// The host routines run on x86-64, where a NaN operand propagates with its
// sign (the first operand's when both are NaN) and an invalid operation
// (Inf * 0, Inf - Inf) yields the negative default NaN; the host fp16 rule
// then keeps that sign on the resulting infinity.  AMD hardware makes
// positive default NaNs, so NaN results get their host sign explicitly.
// (Only reachable when a block's d or dmin is Inf or NaN.)
__device__ __forceinline__ float host_nan(bool negative) {
    return __builtin_bit_cast(float, negative ? 0xffc00000u : 0x7fc00000u);
}

// element e of a Q4_K block (kernels.cu:209-230)
__device__ __forceinline__ float q4k_value(const uint8_t* blk, int e) {
    const int j = e >> 6, hi = (e & 63) >= 32;
    const int g = 2 * j + hi;
    const uint8_t* s = blk + 4;
    int sc, m;
    if (g < 4) {
        sc = s[g] & 63;
        m = s[g + 4] & 63;
    } else {
        sc = (s[g + 4] & 0x0f) | ((s[g - 4] >> 6) << 4);
        m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
    }
    const uint8_t b = blk[16 + 32 * j + (e & 31)];
    const int q = hi ? (b >> 4) : (b & 0x0f);
    const float d = blk_half(blk), dmin = blk_half(blk + 2);
    const float v = d * (float)sc * (float)q - dmin * (float)m;
    if (!__builtin_isnan(v)) return v;
    // host order: (d*sc)*q - dmin*m
    if (__builtin_isnan(d)) return host_nan(__builtin_signbit(d));
    if (__builtin_isinf(d) && (sc == 0 || q == 0)) return host_nan(true);
    if (__builtin_isnan(dmin)) return host_nan(__builtin_signbit(dmin));
    return host_nan(true);   // dmin*0 with dmin = Inf, or Inf - Inf
}

// element e of a Q6_K block (kernels.cu:134-172)
__device__ __forceinline__ float q6k_value(const uint8_t* blk, int e) {
    const int h = e >> 7, part = (e & 127) >> 5, i = e & 31;
    const uint8_t lb = blk[64 * h + 32 * (part & 1) + i];
    const int lo = part < 2 ? (lb & 0x0f) : (lb >> 4);
    const int hi2 = (blk[128 + 32 * h + i] >> (2 * part)) & 3;
    const int q = (lo | (hi2 << 4)) - 32;
    const int8_t sc = (int8_t)blk[192 + 8 * h + i / 16 + 2 * part];
    const float d = blk_half(blk + 208);
    const float v = d * (float)sc * (float)q;
    if (!__builtin_isnan(v)) return v;
    return host_nan(__builtin_isnan(d) ? __builtin_signbit(d) : true);   // NaN d, or Inf * 0
}

// The token comes from `token_at` (device memory) when that is not null; a
// token there outside [0, vocab) yields a zero row instead of a read past
// the table (the host validates the scalar form).
__global__ void embed_q6k_kernel(const uint8_t* __restrict__ table, int32_t token_id,
                                 const int32_t* __restrict__ token_at, int vocab, uint16_t* __restrict__ out,
                                 int hidden) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= hidden) return;
    if (token_at) {
        token_id = *token_at;
        if (token_id < 0 || token_id >= vocab) {
            out[idx] = 0;
            return;
        }
    }
    const size_t nb = (size_t)hidden / kQK;
    const uint8_t* row = table + (size_t)token_id * nb * kQ6KBytes;
    out[idx] = f2h_rne(q6k_value(row + (size_t)(idx / kQK) * kQ6KBytes, idx % kQK));
}

template <int kKind>
__global__ void dequant_kernel(const uint8_t* __restrict__ w, uint64_t count, uint16_t* __restrict__ out) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        const uint64_t b = i / kQK;
        const int e = (int)(i % kQK);
        float v;
        if constexpr (kKind == 4) {
            v = q4k_value(w + b * kQ4KBytes, e);
        } else {
            v = q6k_value(w + b * kQ6KBytes, e);
        }
        out[i] = f2h_ties_away(v);
    }
}

}  // namespace

hipError_t launch_embed_q6k(const uint8_t* table, int32_t token_id, const int32_t* token_at, int vocab,
                            uint16_t* out, int hidden, hipStream_t s) {
    const int block = 256;
    launch_kernel(embed_q6k_kernel, dim3((hidden + block - 1) / block), dim3(block), 0, s, table, token_id,
                  token_at, vocab, out, hidden);
    return hipGetLastError();
}

static dim3 dequant_grid(uint64_t count) {
    uint64_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    return dim3((unsigned)blocks);
}

hipError_t launch_dequant_q4k_f16(const uint8_t* w, uint64_t count, uint16_t* out, hipStream_t s) {
    const dim3 g = dequant_grid(count);
    launch_kernel(dequant_kernel<4>, g, dim3(256), 0, s, w, count, out);
    return hipGetLastError();
}

hipError_t launch_dequant_q6k_f16(const uint8_t* w, uint64_t count, uint16_t* out, hipStream_t s) {
    const dim3 g = dequant_grid(count);
    launch_kernel(dequant_kernel<6>, g, dim3(256), 0, s, w, count, out);
    return hipGetLastError();
}

}  // namespace citlali::hip
