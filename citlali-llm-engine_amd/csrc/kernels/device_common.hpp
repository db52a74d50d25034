// device_common.hpp -- small device helpers shared by the gfx950 kernels.
//
// All kernels are written for CDNA4 wave64.  fp16 values travel as uint16_t
// bit patterns (the reference's convention, kernels.h:8-61).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace citlali::hip {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Vectors the compiler may only assume 2-byte aligned: Q6_K super-blocks start
// on 2-byte boundaries and are read with unaligned global loads.
typedef u32x4 u32x4_a2 __attribute__((aligned(2)));
typedef u32x2 u32x2_a2 __attribute__((aligned(2)));

constexpr int kWave = 64;
constexpr int kQK = 256;          // values per K-quant super-block
constexpr int kQ4KBytes = 144;    // d, dmin, scales[12], qs[128]
constexpr int kQ6KBytes = 210;    // ql[128], qh[64], scales[16], d

__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Nearest-even fp32 -> fp16 (v_cvt_f16_f32 under the default round mode):
// the rule of the reference's device stores (__float2half, kernels.cu:21-24).
__device__ __forceinline__ uint16_t f2h_rne(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// The reference's host rule (dtype.cpp:136-176): nearest with ties away from
// zero, NaN and overflow -> signed Inf, |x| < 2^-25 -> signed zero.  Used
// where device output must equal the host dequant routines bit for bit.
__device__ __forceinline__ uint16_t f2h_ties_away(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    const uint32_t s = (u >> 16) & 0x8000u;
    const int e16 = static_cast<int>((u >> 23) & 0xffu) - 112;
    const uint32_t frac = u & 0x7fffffu;
    uint32_t h;
    if (e16 >= 31) {
        h = 0x7c00u;
    } else if (e16 > 0) {
        h = ((static_cast<uint32_t>(e16) << 10) | (frac >> 13)) + ((frac >> 12) & 1u);
    } else if (e16 < -10) {
        h = 0u;
    } else {
        const uint32_t sig = frac | 0x800000u;
        const uint32_t sh = static_cast<uint32_t>(14 - e16);
        h = (sig >> sh) + ((sig >> (sh - 1u)) & 1u);
    }
    return static_cast<uint16_t>(s | h);
}

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

// v_dot2_f32_f16: a.x*b.x + a.y*b.y + c with fp32 accumulation.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// ---- cross-lane moves on the VALU (DPP and permlane swaps, no LDS) ----
// DPP controls (GFX9 encoding)
constexpr int kDppXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;     // quad_perm [2,3,0,1]
template <int N>
struct DppRor { static constexpr int value = 0x120 + N; };   // row_ror:N (N = 1..15)
constexpr int kDppMirror = 0x140;       // row_mirror: lane i <-> 15 - i of each 16
constexpr int kDppHalfMirror = 0x141;   // row_half_mirror: lane i <-> 7 - i of each 8

template <int Ctrl>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), Ctrl, 0xF, 0xF, false));
}
// Permlane swaps: v_permlane16_swap exchanges the odd 16-lane rows of its
// first operand with the even rows of its second, v_permlane32_swap lanes
// 32-63 of the first with lanes 0-31 of the second.  Called with a = b = v,
// afterwards {a, b} holds v and its lane ^ 16 (^ 32) partner in every lane,
// so a + b and max(a, b) are the pairwise reductions, on the VALU.  Inline
// asm because this compiler reads the builtins' second result back as the
// first (a + b came out as 2a on the box); s_nop 1 covers the wait states
// between the VALU write of an operand and the permlane read.
__device__ __forceinline__ void swap16(float& a, float& b) {
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float& a, float& b) {
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float sum16(float v) {
    float a = v, b = v;
    swap16(a, b);
    return a + b;
}
__device__ __forceinline__ float sum32(float v) {
    float a = v, b = v;
    swap32(a, b);
    return a + b;
}
__device__ __forceinline__ float max16(float v) {
    float a = v, b = v;
    swap16(a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float max32(float v) {
    float a = v, b = v;
    swap32(a, b);
    return fmaxf(a, b);
}

// Sum over all 64 lanes; every lane gets the same (wave-uniform) result.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<DppRor<4>::value>(v);
    v += dpp<DppRor<8>::value>(v);
    v = sum16(v);
    const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    return lo + hi;
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<DppRor<4>::value>(v));
    v = fmaxf(v, dpp<DppRor<8>::value>(v));
    v = max16(v);
    const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    return fmaxf(lo, hi);
}

// Sum over each group of N consecutive lanes (N = 8, 16 or 32); every lane
// of a group gets the same bits (each step adds a lane's value and its
// partner's, and a + b = b + a).
template <int N>
__device__ __forceinline__ float lane_group_sum(float v) {
    static_assert(N == 8 || N == 16 || N == 32, "group");
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    if constexpr (N >= 16) v += dpp<kDppMirror>(v);
    if constexpr (N == 32) v = sum16(v);
    return v;
}

// Reductions over the lanes that share lane % G (G = 1, 2, 4, 8, 16): the
// 64 / G lanes of one "column"; every lane gets its column's result.
template <int G>
__device__ __forceinline__ float column_sum(float v) {
    if constexpr (G < 2) v += dpp<kDppXor1>(v);
    if constexpr (G < 4) v += dpp<kDppXor2>(v);
    if constexpr (G < 8) v += dpp<DppRor<4>::value>(v);
    if constexpr (G < 16) v += dpp<DppRor<8>::value>(v);
    return sum32(sum16(v));
}
template <int G>
__device__ __forceinline__ float column_max(float v) {
    if constexpr (G < 2) v = fmaxf(v, dpp<kDppXor1>(v));
    if constexpr (G < 4) v = fmaxf(v, dpp<kDppXor2>(v));
    if constexpr (G < 8) v = fmaxf(v, dpp<DppRor<4>::value>(v));
    if constexpr (G < 16) v = fmaxf(v, dpp<DppRor<8>::value>(v));
    return max32(max16(v));
}

// Workgroup barrier that orders LDS only: earlier global loads stay in
// flight across it (a full __syncthreads would wait for them).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- residual add + RMSNorm in runs of eight fp16 values -----------------
// The order shared by add_rms_norm_kernel and the GEMV input prologue: in a
// 256-thread block, thread t owns runs t, t + 256, ...; xs = fp16(x + d)
// (xs = x without d); its sum of squares runs over its runs, then its eight
// values, in order; then wave_sum and the four wave sums in order.
constexpr int kNormThreads = 256;

__device__ __forceinline__ uint32_t add_pair(uint32_t x, uint32_t d) {
    const uint32_t lo = f2h_rne(h2f(x & 0xffffu) + h2f(d & 0xffffu));
    const uint32_t hi = f2h_rne(h2f(x >> 16) + h2f(d >> 16));
    return lo | (hi << 16);
}
__device__ __forceinline__ u32x4 add_run(u32x4 x, u32x4 d, bool has_d) {
    if (!has_d) return x;
    return u32x4{add_pair(x.x, d.x), add_pair(x.y, d.y), add_pair(x.z, d.z), add_pair(x.w, d.w)};
}
__device__ __forceinline__ float sq_pair(uint32_t v, float s) {
#pragma clang fp contract(off)   // the same bits in every kernel that inlines it
    const float a = h2f(v & 0xffffu), b = h2f(v >> 16);
    s += a * a;
    return s + b * b;
}
__device__ __forceinline__ float sq_run(u32x4 v, float s) {
    return sq_pair(v.w, sq_pair(v.z, sq_pair(v.y, sq_pair(v.x, s))));
}
__device__ __forceinline__ uint32_t norm_pair(uint32_t v, uint32_t w, float inv) {
    const uint32_t lo = f2h_rne(h2f(v & 0xffffu) * inv * h2f(w & 0xffffu));
    const uint32_t hi = f2h_rne(h2f(v >> 16) * inv * h2f(w >> 16));
    return lo | (hi << 16);
}
__device__ __forceinline__ u32x4 norm_run(u32x4 v, u32x4 w, float inv) {
    return u32x4{norm_pair(v.x, w.x, inv), norm_pair(v.y, w.y, inv), norm_pair(v.z, w.z, inv),
                 norm_pair(v.w, w.w, inv)};
}
// Sum over the 256 threads; `red` holds 4 floats of LDS.  LDS-only barriers,
// so global loads in flight stay in flight.
__device__ __forceinline__ float norm_block_sum(float s, float* red) {
    s = wave_sum(s);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = s;
    lds_barrier();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

// Head RMSNorm and NeoX RoPE pieces shared by the q/k norm + RoPE + store
// kernel and the attention launch that does the same work in its prologue,
// so both give the same bits.  rsqrt(mean(x^2) + eps) of a 128-dim head whose
// values lie two per lane of a wave (dims l and l + 64): the two 64-lane sums
// added, as a 128-thread block sums them (wave 0 holds dims 0..63).
__device__ __forceinline__ float head_inv_rms(float x_lo, float x_hi, int head_dim, float eps) {
#pragma clang fp contract(off)   // the same bits in every kernel that inlines it
    const float s0 = wave_sum(x_lo * x_lo), s1 = wave_sum(x_hi * x_hi);
    return rsqrtf((s0 + s1) / (float)head_dim + eps);
}

// Pair (i, i + head_dim/2) rotated by position * theta^(-2i/head_dim), each
// result rounded to fp16 (kernels.cu:485-521), in two parts: the angle's
// sine and cosine depend only on the pair and the position, so a caller that
// rotates several heads at one position computes them once.
__device__ __forceinline__ void rope_angle(int i, int head_dim, int position, float theta, float& sn, float& cs) {
#pragma clang fp contract(off)   // the same bits in every kernel that inlines it
    const float inv_freq = powf(theta, -(float)(2 * i) / (float)head_dim);
    const float angle = (float)position * inv_freq;
    sincosf(angle, &sn, &cs);
}
__device__ __forceinline__ void rope_rotate(float x0, float x1, float sn, float cs, uint16_t& y0, uint16_t& y1) {
#pragma clang fp contract(off)
    y0 = f2h_rne(x0 * cs - x1 * sn);
    y1 = f2h_rne(x0 * sn + x1 * cs);
}
__device__ __forceinline__ void rope_pair(float x0, float x1, int i, int head_dim, int position, float theta,
                                          uint16_t& y0, uint16_t& y1) {
    float sn, cs;
    rope_angle(i, head_dim, position, theta, sn, cs);
    rope_rotate(x0, x1, sn, cs, y0, y1);
}

// Orders LDS traffic between lanes of one wave (no workgroup barrier): the
// fence makes earlier LDS writes visible, the wave barrier stops the compiler
// from moving memory operations across this point.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// v unchanged, but only available once `a` and `b` are: a load addressed
// with the result is issued after the code that computes them (an empty asm
// the compiler cannot see through).  The streaming GEMVs refill a register
// slot this way after the dot that reads the slot, so the refill reuses the
// slot's registers instead of fresh ones that the loop edge must copy back
// (the copy waits for the load and drains the pipeline every iteration).
__device__ __forceinline__ int issue_after(int v, float a, float b) {
    asm volatile("" : "+v"(v) : "v"(a), "v"(b));
    return v;
}

// N consecutive floats from LDS (16-byte aligned for N >= 4, 8-byte for 2)
// with the widest reads.
template <int N>
__device__ __forceinline__ void load_floats(const float* p, float (&out)[N]) {
    if constexpr (N == 1) {
        out[0] = p[0];
    } else if constexpr (N == 2) {
        const f32x2 v = *reinterpret_cast<const f32x2*>(p);
        out[0] = v.x;
        out[1] = v.y;
    } else {
        static_assert(N % 4 == 0, "load_floats");
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const f32x4 v = reinterpret_cast<const f32x4*>(p)[i];
            out[4 * i + 0] = v.x;
            out[4 * i + 1] = v.y;
            out[4 * i + 2] = v.z;
            out[4 * i + 3] = v.w;
        }
    }
}

}  // namespace citlali::hip
