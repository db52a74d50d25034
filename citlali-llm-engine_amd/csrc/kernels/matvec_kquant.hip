// matvec_kquant.hip -- fused dequant + GEMV for raw GGUF Q4_K / Q6_K rows.
//
// Semantics follow kernels.cu:195-338 of the reference: y[row] = sum over the
// row's 256-value super-blocks of value(e) * x[256*b + e], where value(e) is
// the exact fp32 dequantised weight (never rounded to fp16) and the sum is
// accumulated in fp32; fp16 outputs are rounded nearest-even.
//
// gfx950 design
//  * Four lanes own one super-block; a wave covers 16 consecutive
//    super-blocks per step.  A Q4_K lane reads the 16-byte header and its
//    32 bytes of quants (group pair j = lane&3) with 128-bit loads; a Q6_K
//    lane (half h, 16-value slice ih) reads its three 16-byte byte ranges
//    through dword-aligned windows, because 210-byte blocks start on 2-byte
//    boundaries.
//  * The block stages x once in LDS, with every run of four values stored as
//    (x0, x2, x1, x3), so that a 32-bit quant word splits into half2 operands
//    with one AND (bytes 0/2) or one shift + AND (bytes 1/3).  Quant codes
//    are placed in the mantissa of an fp16 with a zero exponent (value =
//    code * 2^-24, exact), which v_dot2_f32_f16 multiplies by the matching
//    x pair and accumulates in fp32 -- no per-value int->float conversion.
//  * The per-group offset terms (Q4_K "- dmin*m", Q6_K "- 32") need
//    sum(x) over each group; the block computes those sums while staging x.
//  * No MFMA: M = 1 is not a dense contraction.  The bound is HBM.
#include <algorithm>
#include <type_traits>

#include "device_common.hpp"
#include "launch.hpp"

namespace citlali::hip {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
// Layouts of the x-sum tables the traits read (see stage_x8).
constexpr int kSum32 = 0;     // Q4K: sum over each 32-value group, [b][g]
constexpr int kSumQ6 = 1;     // Q6K: 16-value slices, [b][h][ih][k]
constexpr int kPlain = 2;     // F16: x in its own order, no sums
constexpr int kBatch = 4;        // wave steps whose loads are issued together
// The streaming kernels run two workgroups per CU (two waves per SIMD):
// their register budget is capped to keep both resident.
constexpr int kWavesPerSimd = 2;

// ---------------------------------------------------------------------------
// x staging: permuted fp16 pairs + per-group sums.
// ---------------------------------------------------------------------------

// Permutes one run of eight x values into LDS and writes its share of the
// group sums in the layout kLayout.
template <int kLayout>
__device__ __forceinline__ void stage_x8(const u32x4 raw, int v8, uint32_t* xp, float* sx) {
    if constexpr (kLayout == kPlain) {
        *reinterpret_cast<u32x4*>(xp + (size_t)v8 * 4) = raw;
        return;
    }
    u32x4 perm;
    perm.x = __builtin_amdgcn_perm(raw.y, raw.x, 0x05040100u);
    perm.y = __builtin_amdgcn_perm(raw.y, raw.x, 0x07060302u);
    perm.z = __builtin_amdgcn_perm(raw.w, raw.z, 0x05040100u);
    perm.w = __builtin_amdgcn_perm(raw.w, raw.z, 0x07060302u);
    *reinterpret_cast<u32x4*>(xp + (size_t)v8 * 4) = perm;
    float s = 0.f;
    s += h2f(raw.x & 0xffffu) + h2f(raw.x >> 16);
    s += h2f(raw.y & 0xffffu) + h2f(raw.y >> 16);
    s += h2f(raw.z & 0xffffu) + h2f(raw.z >> 16);
    s += h2f(raw.w & 0xffffu) + h2f(raw.w >> 16);
    if constexpr (kLayout == kSum32) {
        // four consecutive threads hold one 32-value group
        s += dpp<kDppXor1>(s);
        s += dpp<kDppXor2>(s);
        if ((v8 & 3) == 0) sx[v8 >> 2] = s;
    } else {
        // two consecutive threads hold one 16-value slice
        s += dpp<kDppXor1>(s);
        if ((v8 & 1) == 0) {
            const int v = v8 * 8;
            const int b = v >> 8, in = v & 255;
            const int h = in >> 7, k = (in & 127) >> 5, ih = (in & 31) >> 4;
            sx[b * 16 + h * 8 + ih * 4 + k] = s;
        }
    }
}

// x staging split in two so its global loads can be issued before the weight
// loads: vmcnt retires loads in order, so x issued last would wait for every
// weight load.  kRuns = K / 8 runs of eight values; thread t stages runs
// t, t + kBlock, ... (kIter per thread; when kRuns is not a multiple of
// kBlock the last pass has whole waves without a run, which hold zeros).
// kNorm: the staged input is the residual add + RMSNorm of x (NormIn, in the
// run order of device_common.hpp; d, w and xs_out 16-byte aligned), its
// loads issued with x's; `red` is 4 floats of LDS.
template <int kLayout, int kRuns, bool kNorm = false>
struct XStage {
    static constexpr int kIter = (kRuns + kBlock - 1) / kBlock;
    static_assert(kRuns % kWave == 0, "whole waves of runs");
    u32x4 raw[kIter];
    u32x4 dr[kNorm ? kIter : 1], wr[kNorm ? kIter : 1];
    __device__ static __forceinline__ bool has_run(int i) {
        return kRuns % kBlock == 0 || i * kBlock + (int)threadIdx.x < kRuns;
    }
    // run index of pass i (a thread without a run re-reads its first one)
    __device__ static __forceinline__ size_t run_of(int i) {
        return has_run(i) ? (size_t)i * kBlock + threadIdx.x : (size_t)threadIdx.x;
    }
    __device__ static __forceinline__ u32x4 keep(u32x4 v, int i) {
        if (has_run(i)) return v;
        return u32x4{0u, 0u, 0u, 0u};   // zeros: add nothing to the sum of squares
    }
    __device__ __forceinline__ void load(const uint16_t* __restrict__ x, const NormIn& n) {
#pragma unroll
        for (int i = 0; i < kIter; ++i) raw[i] = *reinterpret_cast<const u32x4*>(x + run_of(i) * 8);
        if constexpr (kNorm) {
            // branch-free: without d the loads re-read x (unused)
            const uint16_t* dp = n.d ? n.d : x;
#pragma unroll
            for (int i = 0; i < kIter; ++i) {
                dr[i] = *reinterpret_cast<const u32x4*>(dp + run_of(i) * 8);
                wr[i] = *reinterpret_cast<const u32x4*>(n.w + run_of(i) * 8);
            }
        }
    }
    __device__ __forceinline__ void store(uint32_t* xp, float* sx, float* red, const NormIn& n) {
        if constexpr (kNorm) {
            static_assert(kBlock == kNormThreads, "norm order");
            const bool has_d = n.d != nullptr;
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < kIter; ++i) {
                raw[i] = keep(add_run(raw[i], dr[i], has_d), i);
                s = sq_run(raw[i], s);
            }
            if (n.xs_out && blockIdx.x == 0) {
#pragma unroll
                for (int i = 0; i < kIter; ++i)
                    if (has_run(i))
                        *reinterpret_cast<u32x4*>(n.xs_out + ((size_t)i * kBlock + threadIdx.x) * 8) = raw[i];
            }
            s = norm_block_sum(s, red);
            const float inv = rsqrtf(s / (float)(kRuns * 8) + n.eps);
#pragma unroll
            for (int i = 0; i < kIter; ++i) raw[i] = norm_run(raw[i], wr[i], inv);
        }
#pragma unroll
        for (int i = 0; i < kIter; ++i)
            if (has_run(i)) stage_x8<kLayout>(raw[i], i * kBlock + threadIdx.x, xp, sx);   // wave-uniform
        lds_barrier();
    }
};

// Any K (a multiple of 256): every thread stages runs v8 = tid, tid + 256, ...
// (a multiple of 4 runs per thread keeps each group's runs on consecutive
// threads of one pass).
template <int kLayout>
__device__ __forceinline__ void stage_x(const uint16_t* __restrict__ x, int K, uint32_t* xp, float* sx) {
    const int n8 = K >> 3;
    for (int v8 = threadIdx.x; v8 < n8; v8 += kBlock)
        stage_x8<kLayout>(*reinterpret_cast<const u32x4*>(x + (size_t)v8 * 8), v8, xp, sx);
    lds_barrier();
}

// ---------------------------------------------------------------------------
// Q4_K: d(f16) dmin(f16) scales[12] qs[128]   (weight_loader.cpp:150-161)
// ---------------------------------------------------------------------------
struct Q4K {
    static constexpr int kBytes = kQ4KBytes;
    static constexpr int kSxPerBlock = 8;
    static constexpr int kSumLayout = kSum32;
    static constexpr int kLanesPerSb = 4;
    static constexpr int kSbPerStep = kWave / kLanesPerSb;
    static constexpr int kHoistSteps = 4;   // x held in registers for rows of up to this many steps
    static constexpr int kMaxSteps = 7;     // longest row a wave streams (K = 25600)
    struct Frag { u32x4 hdr, q0, q1; };

    __device__ static __forceinline__ Frag load(const uint8_t* sb, int j) {
        Frag f;
        f.hdr = *reinterpret_cast<const u32x4*>(sb);
        f.q0 = *reinterpret_cast<const u32x4*>(sb + 16 + 32 * j);
        f.q1 = *reinterpret_cast<const u32x4*>(sb + 32 + 32 * j);
        return f;
    }

    // The x values lane j needs for super-block b (its 64 staged values and
    // the two 32-value sums); loop-invariant across rows, so the streaming
    // loops load them into registers once.
    struct XRegs { u32x4 l[4], h[4]; f32x2 s; };
    __device__ static __forceinline__ XRegs xload(const uint32_t* xp, const float* sx, int j, int b) {
        const uint32_t* xl = xp + ((b * kQK + 64 * j) >> 1);
        XRegs r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r.l[i] = *reinterpret_cast<const u32x4*>(xl + 4 * i);
            r.h[i] = *reinterpret_cast<const u32x4*>(xl + 16 + 4 * i);
        }
        r.s = *reinterpret_cast<const f32x2*>(sx + b * 8 + 2 * j);
        return r;
    }
    __device__ static __forceinline__ float dot(const Frag& f, int j, const uint32_t* xp, const float* sx, int b) {
        return dot(f, j, xload(xp, sx, j, b));
    }

    // Contribution of lane j (group pair 2j, 2j+1) of a super-block.
    __device__ static __forceinline__ float dot(const Frag& f, int j, const XRegs& x) {
        // no fused multiply-adds: every kernel that inlines this computes the
        // same bits (the fused launches equal the plain ones)
#pragma clang fp contract(off)
        // 6-bit (scale, min) codes of groups 2j, 2j+1 (kernels.cu:174-186):
        // work on the two bytes k, k+1 of each 4-byte scale word at once.
        const uint32_t sh = (uint32_t)((2 * j) & 3) * 8u;
        const uint32_t a = (f.hdr.y >> sh) & 0xffffu;   // scales[k], [k+1]
        const uint32_t bq = (f.hdr.z >> sh) & 0xffffu;  // scales[k+4], [k+5]
        const uint32_t c = (f.hdr.w >> sh) & 0xffffu;   // scales[k+8], [k+9]
        uint32_t sc, mn;
        if (j < 2) {
            sc = a & 0x3f3fu;
            mn = bq & 0x3f3fu;
        } else {
            sc = (c & 0x0f0fu) | ((a >> 2) & 0x3030u);
            mn = ((c >> 4) & 0x0f0fu) | ((bq >> 2) & 0x3030u);
        }
        const float d = h2f(f.hdr.x & 0xffffu);
        const float dmin = h2f(f.hdr.x >> 16);

        const u32x4 xl0 = x.l[0], xl1 = x.l[1], xl2 = x.l[2], xl3 = x.l[3];
        const u32x4 xh0 = x.h[0], xh1 = x.h[1], xh2 = x.h[2], xh3 = x.h[3];
        const uint32_t q[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
        const uint32_t XL[16] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w,
                                 xl2.x, xl2.y, xl2.z, xl2.w, xl3.x, xl3.y, xl3.z, xl3.w};
        const uint32_t XH[16] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w,
                                 xh2.x, xh2.y, xh2.z, xh2.w, xh3.x, xh3.y, xh3.z, xh3.w};
        float plo = 0.f, phi = 0.f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t w = q[t];
            const uint32_t w8 = w >> 8;
            plo = dot2(w & 0x000f000fu, XL[2 * t], plo);       // q * 2^-24
            plo = dot2(w8 & 0x000f000fu, XL[2 * t + 1], plo);
            phi = dot2(w & 0x00f000f0u, XH[2 * t], phi);       // q * 2^-20
            phi = dot2(w8 & 0x00f000f0u, XH[2 * t + 1], phi);
        }
        const f32x2 s = x.s;
        const float a_lo = d * (float)(sc & 0xffu) * 16777216.0f;
        const float a_hi = d * (float)(sc >> 8) * 1048576.0f;
        const float m_lo = dmin * (float)(mn & 0xffu);
        const float m_hi = dmin * (float)(mn >> 8);
        return (a_lo * plo - m_lo * s.x) + (a_hi * phi - m_hi * s.y);
    }
};

// ---------------------------------------------------------------------------
// Q6_K: ql[128] qh[64] scales int8[16] d(f16)   (weight_loader.cpp:247-257)
// ---------------------------------------------------------------------------
struct Q6K {
    static constexpr int kBytes = kQ6KBytes;
    static constexpr int kSxPerBlock = 16;
    static constexpr int kSumLayout = kSumQ6;
    static constexpr int kLanesPerSb = 4;
    static constexpr int kSbPerStep = kWave / kLanesPerSb;
    static constexpr int kHoistSteps = 4;
    static constexpr int kMaxSteps = 7;
    struct Frag { uint32_t wa[4], wb[4], u[4]; uint32_t s0, s1, dbits; };

    // lane_in_sb = 2*h + ih.  A 210-byte block starts on a 2-byte boundary;
    // gfx950 global loads take unaligned addresses (the ROCm default
    // unaligned mode, which the compiler targets), so each range is one
    // 16-byte load.
    __device__ static __forceinline__ Frag load(const uint8_t* sb, int l4) {
        const int h = l4 >> 1, ih = l4 & 1;
        Frag f;
        const u32x4 a = *reinterpret_cast<const u32x4_a2*>(sb + 64 * h + 16 * ih);        // ql, low
        const u32x4 b = *reinterpret_cast<const u32x4_a2*>(sb + 64 * h + 32 + 16 * ih);   // ql, high
        const u32x4 c = *reinterpret_cast<const u32x4_a2*>(sb + 128 + 32 * h + 16 * ih);  // qh
        const u32x2 sc = *reinterpret_cast<const u32x2_a2*>(sb + 192 + 8 * h);           // scales
        f.wa[0] = a.x; f.wa[1] = a.y; f.wa[2] = a.z; f.wa[3] = a.w;
        f.wb[0] = b.x; f.wb[1] = b.y; f.wb[2] = b.z; f.wb[3] = b.w;
        f.u[0] = c.x; f.u[1] = c.y; f.u[2] = c.z; f.u[3] = c.w;
        f.s0 = sc.x;
        f.s1 = sc.y;
        f.dbits = *reinterpret_cast<const uint16_t*>(sb + 208);
        return f;
    }

    // The x values lane l4 needs for super-block b: slice k, pair t of its
    // 16 positions per slice, and the four slice sums (loop-invariant).
    struct XRegs { u32x2 v[4][4]; f32x4 s; };
    __device__ static __forceinline__ XRegs xload(const uint32_t* xp, const float* sx, int l4, int b) {
        const int h = l4 >> 1, ih = l4 & 1;
        // x pairs of slice k: values 128h + 32k + 16ih + [0,16)
        const uint32_t* xb = xp + ((b * kQK + 128 * h + 16 * ih) >> 1);
        XRegs r;
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int t = 0; t < 4; ++t) r.v[k][t] = *reinterpret_cast<const u32x2*>(xb + k * 16 + 2 * t);
        r.s = *reinterpret_cast<const f32x4*>(sx + b * 16 + h * 8 + ih * 4);
        return r;
    }
    __device__ static __forceinline__ float dot(const Frag& f, int l4, const uint32_t* xp, const float* sx, int b) {
        return dot(f, l4, xload(xp, sx, l4, b));
    }

    __device__ static __forceinline__ float dot(const Frag& f, int l4, const XRegs& x) {
#pragma clang fp contract(off)   // the same bits in every kernel that inlines it
        const int ih = l4 & 1;
        const float d = h2f((uint16_t)f.dbits);
        // int8 scales sc[8h + ih + 2k], k = 0..3 (kernels.cu:166-167)
        // (int8_t casts: the result must be converted as a signed value)
        const uint32_t sh = (uint32_t)ih * 8u;
        const float sc0 = (float)(int8_t)(f.s0 >> sh);
        const float sc1 = (float)(int8_t)(f.s0 >> (sh + 16u));
        const float sc2 = (float)(int8_t)(f.s1 >> sh);
        const float sc3 = (float)(int8_t)(f.s1 >> (sh + 16u));

        float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t wa = f.wa[t], wb = f.wb[t], u = f.u[t];
            // 6-bit codes of the word's four bytes for each slice k: low
            // nibble (ql) | the slice's two qh bits << 4, one byte each;
            // then bytes 0/2 and bytes 1/3 go to the two fp16 halves of a
            // dot2 operand (one byte permute each, the other bytes zero).
            const uint32_t k0 = (wa & 0x0f0f0f0fu) | ((u << 4) & 0x30303030u);
            const uint32_t k1 = (wb & 0x0f0f0f0fu) | ((u << 2) & 0x30303030u);
            const uint32_t k2 = ((wa >> 4) & 0x0f0f0f0fu) | (u & 0x30303030u);
            const uint32_t k3 = ((wb >> 4) & 0x0f0f0f0fu) | ((u >> 2) & 0x30303030u);
            constexpr uint32_t kEven = 0x0c020c00u, kOdd = 0x0c030c01u;   // 0x0c selects a zero byte
            const uint32_t c0a = __builtin_amdgcn_perm(0u, k0, kEven), c0b = __builtin_amdgcn_perm(0u, k0, kOdd);
            const uint32_t c1a = __builtin_amdgcn_perm(0u, k1, kEven), c1b = __builtin_amdgcn_perm(0u, k1, kOdd);
            const uint32_t c2a = __builtin_amdgcn_perm(0u, k2, kEven), c2b = __builtin_amdgcn_perm(0u, k2, kOdd);
            const uint32_t c3a = __builtin_amdgcn_perm(0u, k3, kEven), c3b = __builtin_amdgcn_perm(0u, k3, kOdd);
            const u32x2 x0 = x.v[0][t], x1 = x.v[1][t], x2 = x.v[2][t], x3 = x.v[3][t];
            p0 = dot2(c0b, x0.y, dot2(c0a, x0.x, p0));
            p1 = dot2(c1b, x1.y, dot2(c1a, x1.x, p1));
            p2 = dot2(c2b, x2.y, dot2(c2a, x2.x, p2));
            p3 = dot2(c3b, x3.y, dot2(c3a, x3.x, p3));
        }
        const f32x4 s = x.s;
        // sum (q6 - 32) x = 2^24 P - 32 S
        const float t0 = sc0 * (p0 * 16777216.0f - 32.0f * s.x);
        const float t1 = sc1 * (p1 * 16777216.0f - 32.0f * s.y);
        const float t2 = sc2 * (p2 * 16777216.0f - 32.0f * s.z);
        const float t3 = sc3 * (p3 * 16777216.0f - 32.0f * s.w);
        return d * ((t0 + t1) + (t2 + t3));
    }
};

// ---------------------------------------------------------------------------
// F16: fp16 weights (the DequantizeToFp16 path, kernels.cu:27-35, 381-412),
// seen as 512-byte blocks of 256 values so that the streaming kernels below
// serve them too.  Lane j of a block reads bytes 16 j + 64 i, i = 0..7:
// every load instruction of a wave covers 64 contiguous bytes of each of
// its 16 blocks.  x is staged in its own order; a weight word (two fp16)
// meets the matching x word in one v_dot2_f32_f16.
// ---------------------------------------------------------------------------
struct F16 {
    static constexpr int kBytes = 2 * kQK;
    static constexpr int kSxPerBlock = 0;
    static constexpr int kSumLayout = kPlain;
    static constexpr int kLanesPerSb = 4;
    static constexpr int kSbPerStep = kWave / kLanesPerSb;
    // a lane's x is 32 registers per step: rows of four steps read it from
    // LDS instead
    static constexpr int kHoistSteps = 3;
    // 32 registers of weights per step in flight: longer rows take the flat
    // kernel
    static constexpr int kMaxSteps = 4;
    struct Frag { u32x4 v[8]; };

    __device__ static __forceinline__ Frag load(const uint8_t* sb, int j) {
        Frag f;
#pragma unroll
        for (int i = 0; i < 8; ++i) f.v[i] = *reinterpret_cast<const u32x4*>(sb + 16 * j + 64 * i);
        return f;
    }

    struct XRegs { u32x4 v[8]; };
    __device__ static __forceinline__ XRegs xload(const uint32_t* xp, const float*, int j, int b) {
        const uint32_t* xb = xp + ((b * kQK + 8 * j) >> 1);
        XRegs r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r.v[i] = *reinterpret_cast<const u32x4*>(xb + 16 * i);
        return r;
    }
    __device__ static __forceinline__ float dot(const Frag& f, int j, const uint32_t* xp, const float* sx, int b) {
        return dot(f, j, xload(xp, sx, j, b));
    }

    // Sum over lane j's 64 values of the block: four fp32 partial chains
    // (one per word of a 16-byte load), added in a fixed order.
    __device__ static __forceinline__ float dot(const Frag& f, int, const XRegs& x) {
#pragma clang fp contract(off)
        float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            p0 = dot2(f.v[i].x, x.v[i].x, p0);
            p1 = dot2(f.v[i].y, x.v[i].y, p1);
            p2 = dot2(f.v[i].z, x.v[i].z, p2);
            p3 = dot2(f.v[i].w, x.v[i].w, p3);
        }
        return (p0 + p1) + (p2 + p3);
    }
};

template <bool kF32>
__device__ __forceinline__ void store_y(void* y, int row, float v) {
    if constexpr (kF32) {
        static_cast<float*>(y)[row] = v;
    } else {
        static_cast<uint16_t*>(y)[row] = f2h_rne(v);
    }
}

// Up to three matrices of one type that read the same x, seen as one row
// space: row r is row r - end[s-1] of matrix s, the first s with r < end[s]
// (end[] cumulative; unused entries repeat the total, end[2]).
struct RowSet {
    const uint8_t* w[3];
    void* y[3];
    int end[3];
};

// Rows per wave step for rows of nb super-blocks (`per_step` blocks a step).
__host__ __device__ constexpr int pack_rows(int nb, int per_step) {
    return (nb > 0 && nb < per_step && per_step % nb == 0) ? per_step / nb : 1;
}

// Rows packed per wave step: rows of NB blocks, NB dividing the 16 blocks of
// a step (4 or 8: Qwen3-0.6B / 1.7B hidden sizes), take 16 / NB rows per
// step, lane group sub / NB reading block sub % NB of its own row; other row
// lengths take one row per step.  A "unit" is the rows one step covers.
template <class QT, int NB>
struct Pack {
    static constexpr int P = pack_rows(NB, QT::kSbPerStep);
    static constexpr int kGroupLanes = P > 1 ? NB * QT::kLanesPerSb : kWave;   // lanes summing one row
    __host__ __device__ static constexpr int units(int rows) { return (rows + P - 1) / P; }
    // the row of unit u that lane group `sub` works on
    __device__ static __forceinline__ int row(int u, int sub) { return P > 1 ? u * P + sub / NB : u; }
    // a row's sum over its lanes; with packing, lanes of one row only
    __device__ static __forceinline__ float reduce(float v) {
        if constexpr (P > 1) return lane_group_sum<kGroupLanes>(v);
        else return wave_sum(v);
    }
    // the lane that stores its row's result
    __device__ static __forceinline__ bool leader(int lane) { return lane % kGroupLanes == 0; }
};

// Rows of 16*S super-blocks, streamed: each wave walks units gw, gw + W, ...
// (W = waves walking this row set; a unit is one row, or 16 / NB rows of a
// short length, see Pack), a unit being S steps of 16 super-blocks, and
// keeps the next D = S*M steps' fragments in flight while it computes the
// current one (a ring of D register slots, indices fixed at compile time by
// unrolling M units).  x is loaded before the first fragments and staged in
// LDS behind them.  Loads are branch-free (rows past the end re-read the
// last row).  kSegs = 1 reads only w[0] / y[0].  kRefill = false: the wave
// computes its M units (all loaded up front) and stops; the grid then has
// M * W >= units.  NB (an even block count that is not a multiple of 16,
// S = ceil(NB / 16)): rows ending in a partial wave step; unless NB packs,
// the lanes of blocks NB.. in that step load block NB - 1 (in bounds) and add
// nothing.
template <class QT, bool kF32, int S, int M, int kSegs, bool kRefill = true, bool kNorm = false, int NB = 0>
__device__ __forceinline__ void stream_rows(const RowSet& rs, const uint16_t* __restrict__ x, int K, uint8_t* smem,
                                            int gw, int W, const NormIn& nrm) {
    static_assert(NB == 0 || (NB % 2 == 0 && (NB + QT::kSbPerStep - 1) / QT::kSbPerStep == S), "partial last step");
    using PK = Pack<QT, NB>;
    constexpr int nb = NB ? NB : S * QT::kSbPerStep;   // K = 256 nb
    uint32_t* xp = reinterpret_cast<uint32_t*>(smem);
    float* sx = reinterpret_cast<float*>(smem + (size_t)K * 2);
    const int N = rs.end[kSegs - 1];
    const int U = PK::units(N);

    const int lane = threadIdx.x & (kWave - 1);
    const int l4 = lane % QT::kLanesPerSb;
    const int sub = lane / QT::kLanesPerSb;
    // block of step t this lane reads; false: past the row end (adds nothing)
    auto blk = [&](int t) {
        if constexpr (PK::P > 1) return sub % NB;
        else return NB ? min(t * QT::kSbPerStep + sub, nb - 1) : t * QT::kSbPerStep + sub;
    };
    auto live = [&](int t) { return NB == 0 || PK::P > 1 || t * QT::kSbPerStep + sub < nb; };
    constexpr int D = S * M;

    // matrix of row r and r's first row index in it
    auto seg_of = [&](int r) { return kSegs == 1 ? 0 : (int)(r >= rs.end[0]) + (int)(r >= rs.end[1]); };
    auto seg_base = [&](int sg) { return sg == 0 ? 0 : sg == 1 ? rs.end[0] : rs.end[1]; };
    auto frag_at = [&](int unit, int t) {
        const int r = min(PK::row(unit, sub), N - 1);
        const int sg = seg_of(r);
        const uint8_t* w = sg == 0 ? rs.w[0] : sg == 1 ? rs.w[1] : rs.w[2];
        const size_t f = (size_t)(r - seg_base(sg)) * nb + blk(t);
        return QT::load(w + f * QT::kBytes, l4);
    };

    XStage<QT::kSumLayout, nb * 32, kNorm> xs;   // K / 8 = 32 nb runs of eight values
    xs.load(x, nrm);
    __builtin_amdgcn_sched_barrier(0);   // issue order: x, first fragments, staging
    typename QT::Frag fr[D];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int t = 0; t < S; ++t) {
            fr[m * S + t] = frag_at(gw + m * W, t);
            __builtin_amdgcn_sched_barrier(0);   // slot order, as the refills below
        }
    xs.store(xp, sx, sx + nb * QT::kSxPerBlock, nrm);
    constexpr bool kHoist = S <= QT::kHoistSteps;
    typename QT::XRegs xr[kHoist ? S : 1];   // this lane's x, the same for every row
    if constexpr (kHoist) {
#pragma unroll
        for (int t = 0; t < S; ++t) xr[t] = QT::xload(xp, sx, l4, blk(t));
    }

    for (int unit = gw; unit < U; unit += M * W) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const int u = unit + m * W;
            float acc = 0.f;
#pragma unroll
            for (int t = 0; t < S; ++t) {
                float c = kHoist ? QT::dot(fr[m * S + t], l4, xr[kHoist ? t : 0])
                                 : QT::dot(fr[m * S + t], l4, xp, sx, blk(t));
                if (NB != 0 && t == S - 1) c = live(t) ? c : 0.f;
                acc += c;
                // Refill after the dot has read the slot (issue_after), in
                // slot order (vmcnt retires loads in issue order: a reordered
                // refill would make the next slot's wait cover it).
                if constexpr (kRefill) {
                    fr[m * S + t] = frag_at(issue_after(u + M * W, c, c), t);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            acc = PK::reduce(acc);
            const int r = PK::row(u, sub);
            if (PK::leader(lane) && r < N) {
                const int sg = seg_of(r);
                store_y<kF32>(sg == 0 ? rs.y[0] : sg == 1 ? rs.y[1] : rs.y[2], r - seg_base(sg), acc);
            }
        }
        if constexpr (!kRefill) break;
    }
}

template <class QT, bool kF32, int S, int M, int kSegs, bool kRefill = true, bool kNorm = false, int NB = 0>
__global__ __launch_bounds__(kBlock, kWavesPerSimd) void matvec_stream_kernel(RowSet rs, const uint16_t* __restrict__ x,
                                                                             int K, NormIn nrm) {
    extern __shared__ __align__(16) uint8_t smem[];
    stream_rows<QT, kF32, S, M, kSegs, kRefill, kNorm, NB>(rs, x, K, smem,
                                                           blockIdx.x * kWavesPerBlock + threadIdx.x / kWave,
                                                           gridDim.x * kWavesPerBlock, nrm);
}

// Two row sets of different types in one launch: blocks [0, blocks_a) walk
// set `a` (type QA), the rest walk set `b` (type QB).  Each row is computed
// exactly as the single-matrix launch computes it.
template <class QA, class QB, int S, int M, bool kRefill = true, bool kNorm = false, int NB = 0>
__global__ __launch_bounds__(kBlock, kWavesPerSimd) void matvec_group_kernel(RowSet a, RowSet b, int blocks_a,
                                                                            const uint16_t* __restrict__ x, int K,
                                                                            NormIn nrm) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int wave = threadIdx.x / kWave;
    if ((int)blockIdx.x < blocks_a)
        stream_rows<QA, false, S, M, 3, kRefill, kNorm, NB>(a, x, K, smem, blockIdx.x * kWavesPerBlock + wave,
                                                            blocks_a * kWavesPerBlock, nrm);
    else
        stream_rows<QB, false, S, M, 3, kRefill, kNorm, NB>(b, x, K, smem,
                                                            (blockIdx.x - blocks_a) * kWavesPerBlock + wave,
                                                            (gridDim.x - blocks_a) * kWavesPerBlock, nrm);
}

// ffn_gate and ffn_up GEMVs plus SwiGLU in one launch (the reference's two
// LinearBackend::forward calls and launch_swiglu, qwen_model.cpp:364-368).
// Each wave computes row r of both matrices exactly as matvec_stream_kernel
// does (same lane mapping and summation order), rounds both to fp16 where
// the separate GEMVs store, and writes act[r] = fp16(silu(g) * u) with the
// swiglu_kernel expression -- the separate launches' results bit for bit.
//
// Rows are handed out at run time.  One workgroup of eight waves per CU
// (two per SIMD) owns a contiguous range of rows; a wave starts on row
// `wave` of the range and takes each further row from an LDS counter when it
// starts the dots of its current one, so the refill goes out as soon as a
// slot is consumed.  A wave whose loads come back earlier computes more rows.
// With two four-wave workgroups per CU and rows fixed in advance, the
// workgroup dispatched second had its loads served after the first one's
// and finished about 2 us later at config 3, the CU running on half its
// waves meanwhile.  Waves 0-3 stage x (the 256-thread order of the other
// GEMVs and of the norm prologue); waves 4-7 only pass the same barriers.
constexpr int kGateUpWaves = 8;
constexpr int kGateUpBlock = kGateUpWaves * kWave;

template <class QT, int S, bool kNorm = false, int NB = 0>
__global__ __launch_bounds__(kGateUpBlock, 2) void matvec_gate_up_kernel(const uint8_t* __restrict__ wg,
                                                                         const uint8_t* __restrict__ wu,
                                                                         const uint16_t* __restrict__ x,
                                                                         uint16_t* __restrict__ act, int K, int N,
                                                                         NormIn nrm) {
    extern __shared__ __align__(16) uint8_t smem[];
    static_assert(NB == 0 || (NB % 2 == 0 && (NB + QT::kSbPerStep - 1) / QT::kSbPerStep == S), "partial last step");
    using PK = Pack<QT, NB>;
    constexpr int nb = NB ? NB : S * QT::kSbPerStep;
    uint32_t* xp = reinterpret_cast<uint32_t*>(smem);
    float* sx = reinterpret_cast<float*>(smem + (size_t)K * 2);
    // the unit counter follows the x tables and the 4 floats of norm scratch
    int* next = reinterpret_cast<int*>(smem + (size_t)nb * kQK * 2 + (size_t)nb * QT::kSxPerBlock * sizeof(float) +
                                       4 * sizeof(float));

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int l4 = lane % QT::kLanesPerSb;
    const int sub = lane / QT::kLanesPerSb;
    auto blk = [&](int t) {
        if constexpr (PK::P > 1) return sub % NB;
        else return NB ? min(t * QT::kSbPerStep + sub, nb - 1) : t * QT::kSbPerStep + sub;
    };
    auto live = [&](int t) { return NB == 0 || PK::P > 1 || t * QT::kSbPerStep + sub < nb; };
    const int U = PK::units(N);
    const int span = (U + (int)gridDim.x - 1) / (int)gridDim.x;
    const int u0 = (int)blockIdx.x * span;
    const int nunits = max(0, min(span, U - u0));

    auto frag_at = [&](const uint8_t* w, int unit, int t) {
        const size_t f = (size_t)min(PK::row(unit, sub), N - 1) * nb + blk(t);
        return QT::load(w + f * QT::kBytes, l4);
    };

    if (threadIdx.x == 0) *next = kGateUpWaves;   // read only after the x barrier
    XStage<QT::kSumLayout, nb * 32, kNorm> xs;   // K = 256 nb
    if (wave < kWavesPerBlock) xs.load(x, nrm);
    __builtin_amdgcn_sched_barrier(0);
    int k = wave;   // this wave's unit u0 + k
    typename QT::Frag fg[S], fu[S];
#pragma unroll
    for (int t = 0; t < S; ++t) {
        fg[t] = frag_at(wg, u0 + k, t);
        fu[t] = frag_at(wu, u0 + k, t);
        __builtin_amdgcn_sched_barrier(0);   // slot order, as the refills below
    }
    if (wave < kWavesPerBlock) {
        xs.store(xp, sx, sx + nb * QT::kSxPerBlock, nrm);
    } else {
        if constexpr (kNorm) lds_barrier();   // norm_block_sum's
        lds_barrier();                        // the staging barrier
    }
    static_assert(S <= QT::kHoistSteps, "gate/up holds x in registers");
    typename QT::XRegs xr[S];   // this lane's x, the same for every row
#pragma unroll
    for (int t = 0; t < S; ++t) xr[t] = QT::xload(xp, sx, l4, blk(t));

    while (k < nunits) {   // wave-uniform
        int kn = 0;
        if (lane == 0) kn = __hip_atomic_fetch_add(next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        kn = __builtin_amdgcn_readfirstlane(kn);
        const bool more = kn < nunits;
        const int unit = u0 + k;
        // Each slot is reloaded with the next row once its dots have read it
        // (issue_after), in slot order.  A one-step row (S = 1) reloads after
        // both dots and skips the reload on its last row; longer rows reload
        // unconditionally (their last row re-reads itself), since a branch
        // there let the compiler move every reload behind the last dot.
        const int un = more ? u0 + kn : unit;
        float ag = 0.f, au = 0.f;
#pragma unroll
        for (int t = 0; t < S; ++t) {
            float cg = QT::dot(fg[t], l4, xr[t]);
            float cu = QT::dot(fu[t], l4, xr[t]);
            if (NB != 0 && t == S - 1) {
                cg = live(t) ? cg : 0.f;
                cu = live(t) ? cu : 0.f;
            }
            ag += cg;
            au += cu;
            if (S > 1 || more) {
                const int nu = issue_after(un, cg, cu);
                fg[t] = frag_at(wg, nu, t);
                fu[t] = frag_at(wu, nu, t);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        ag = PK::reduce(ag);
        au = PK::reduce(au);
        // computed in every lane, so the branch holds only the store (a
        // longer branch region keeps the fragment registers from being
        // reused across rows: the loop edge then copies them and waits for
        // every refill)
        const float g = h2f(f2h_rne(ag)), u = h2f(f2h_rne(au));
        const uint16_t a = f2h_rne(g / (1.0f + expf(-g)) * u);
        const int r = PK::row(unit, sub);
        if (PK::leader(lane) && r < N) act[r] = a;
        k = kn;
    }
}

// Any super-block count: a wave owns kRows rows and walks their super-blocks
// as one flat list; a lane's row is found by multiply-high division.
template <class QT, bool kF32, int kRows>
__global__ __launch_bounds__(kBlock) void matvec_flat_kernel(const uint8_t* __restrict__ w,
                                                             const uint16_t* __restrict__ x,
                                                             void* __restrict__ y, int K, int N,
                                                             uint64_t magic) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint32_t* xp = reinterpret_cast<uint32_t*>(smem);
    float* sx = reinterpret_cast<float*>(smem + (size_t)K * 2);
    stage_x<QT::kSumLayout>(x, K, xp, sx);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int l4 = lane % QT::kLanesPerSb;
    const int sub = lane / QT::kLanesPerSb;
    const int nb = K >> 8;
    const int row0 = (blockIdx.x * kWavesPerBlock + wave) * kRows;
    const int rows = min(kRows, N - row0);
    const int nflat = rows > 0 ? rows * nb : 0;

    float acc[kRows];
#pragma unroll
    for (int k = 0; k < kRows; ++k) acc[k] = 0.f;

    for (int f0 = 0; f0 < nflat; f0 += kBatch * QT::kSbPerStep) {
        typename QT::Frag fr[kBatch];
        int rl[kBatch], bl[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const uint32_t f = (uint32_t)(f0 + u * QT::kSbPerStep + sub);
            const uint32_t r = (uint32_t)(((uint64_t)f * magic) >> 32);
            rl[u] = (int)f < nflat ? (int)r : -1;
            bl[u] = (int)(f - r * (uint32_t)nb);
            if (rl[u] >= 0) fr[u] = QT::load(w + ((size_t)row0 * nb + f) * QT::kBytes, l4);
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (rl[u] >= 0) {
                const float c = QT::dot(fr[u], l4, xp, sx, bl[u]);
#pragma unroll
                for (int k = 0; k < kRows; ++k) acc[k] += (rl[u] == k) ? c : 0.f;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
        const float s = wave_sum(acc[k]);
        if (lane == 0 && k < rows) store_y<kF32>(y, row0 + k, s);
    }
}

int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

// `per_cu` workgroups per CU (two: two waves per SIMD), never more waves than
// rows.
int stream_grid(int rows, int per_cu = 2) {
    const int grid = per_cu * device_cus();
    const int need = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
    return grid > need ? need : grid;
}

// K = 256 nb, nb = NB (short rows) or 16 S.  Rows of two or more wave steps
// run one workgroup per CU: ffn_down at config 3 (Q6_K, 48 super-blocks, two
// rows per wave with two workgroups per CU) measured 9.5 us this way against
// 9.7-10.4 us with two, whose second workgroup has its loads served after the
// first's and finishes last.
template <class QT, bool kF32, int S, int M, int kSegs, bool kNorm, int NB = 0>
void launch_stream(const RowSet& rs, const uint16_t* x, size_t lds, const NormIn& nrm, hipStream_t stream) {
    constexpr int K = (NB ? NB : S * QT::kSbPerStep) * kQK;
    const int units = Pack<QT, NB>::units(rs.end[kSegs - 1]);
    launch_kernel((matvec_stream_kernel<QT, kF32, S, M, kSegs, true, kNorm, NB>),
                  dim3(stream_grid(units, S >= 2 ? 1 : 2)), dim3(kBlock), lds, stream, rs, x, K, nrm);
}

// Rows of one wave step (K <= 4096), few rows: every wave loads its M units
// up front and computes them, no refills (M * waves >= units).
template <class QT, bool kF32, int M, int kSegs, bool kNorm, int NB = 0>
void launch_rows_once(const RowSet& rs, const uint16_t* x, size_t lds, const NormIn& nrm, hipStream_t stream) {
    constexpr int K = (NB ? NB : QT::kSbPerStep) * kQK;
    const int units = Pack<QT, NB>::units(rs.end[kSegs - 1]);
    const int grid = (units + M * kWavesPerBlock - 1) / (M * kWavesPerBlock);
    launch_kernel((matvec_stream_kernel<QT, kF32, 1, M, kSegs, false, kNorm, NB>), dim3(grid), dim3(kBlock), lds,
                  stream, rs, x, K, nrm);
}

// Rows ending in a partial wave step (NB blocks, not a multiple of 16).
// Shorter than one step (K = 1024, 2048, 2560, 3072: Qwen3-0.6B / 4B): one
// pass of one unit per wave up to 1024 units, of two up to 4096, streamed
// with one unit in flight beyond (a unit: 16 / NB rows for NB = 4 or 8, one
// row else); longer rows stream with one row in flight.
template <class QT, bool kF32, int kSegs, bool kNorm, int NB>
void launch_partial(const RowSet& rs, const uint16_t* x, size_t lds, const NormIn& nrm, hipStream_t stream) {
    constexpr int S = (NB + QT::kSbPerStep - 1) / QT::kSbPerStep;
    const int rows = Pack<QT, NB>::units(rs.end[kSegs - 1]);
    if constexpr (S == 1) {
        if (rows <= 1024)
            launch_rows_once<QT, kF32, 1, kSegs, kNorm, NB>(rs, x, lds, nrm, stream);
        else if (rows <= 4096)
            launch_rows_once<QT, kF32, 2, kSegs, kNorm, NB>(rs, x, lds, nrm, stream);
        else
            launch_stream<QT, kF32, 1, 1, kSegs, kNorm, NB>(rs, x, lds, nrm, stream);
    } else {
        launch_stream<QT, kF32, S, 1, kSegs, kNorm, NB>(rs, x, lds, nrm, stream);
    }
}

// K = 4096 S.  Shapes measured on MI355X: at K = 4096 a launch of up to 4096
// rows is fastest as one pass of one, two or four rows per wave (the refill
// loop's loads past the last row cost more than they hide; attn_o, 4096 rows:
// 4.02 us with four rows per wave, 4.31 with two, 4.43 with one); longer
// matrices stream with one row in flight, two once each wave walks at least
// four rows.
template <class QT, bool kF32, int kSegs, bool kNorm = false>
bool launch_stream_for(int nb, const RowSet& rs, const uint16_t* x, size_t lds, const NormIn& nrm,
                       hipStream_t stream) {
    const int rows = rs.end[kSegs - 1];
    switch (nb) {
        case 16:
            if (rows <= 1024)
                launch_rows_once<QT, kF32, 1, kSegs, kNorm>(rs, x, lds, nrm, stream);
            else if (rows <= 3072)
                launch_rows_once<QT, kF32, 2, kSegs, kNorm>(rs, x, lds, nrm, stream);
            else if (rows <= 4096)
                launch_rows_once<QT, kF32, 4, kSegs, kNorm>(rs, x, lds, nrm, stream);
            else if (rows >= 4 * kWavesPerBlock * stream_grid(rows))
                launch_stream<QT, kF32, 1, 2, kSegs, kNorm>(rs, x, lds, nrm, stream);
            else
                launch_stream<QT, kF32, 1, 1, kSegs, kNorm>(rs, x, lds, nrm, stream);
            return true;
        case 32: launch_stream<QT, kF32, 2, 1, kSegs, kNorm>(rs, x, lds, nrm, stream); return true;
        case 48: launch_stream<QT, kF32, 3, 1, kSegs, kNorm>(rs, x, lds, nrm, stream); return true;
        case 64: launch_stream<QT, kF32, 4, 1, kSegs, kNorm>(rs, x, lds, nrm, stream); return true;
        // the other Qwen3 row lengths: hidden 1024 / 2048 / 2560 / 5120, FFN
        // 3072 / 6144 / 9728 / 17408 / 25600 (the last two without the norm
        // prologue, which only hidden-sized inputs take)
        case 4: launch_partial<QT, kF32, kSegs, kNorm, 4>(rs, x, lds, nrm, stream); return true;
        case 8: launch_partial<QT, kF32, kSegs, kNorm, 8>(rs, x, lds, nrm, stream); return true;
        case 10: launch_partial<QT, kF32, kSegs, kNorm, 10>(rs, x, lds, nrm, stream); return true;
        case 12: launch_partial<QT, kF32, kSegs, kNorm, 12>(rs, x, lds, nrm, stream); return true;
        case 20: launch_partial<QT, kF32, kSegs, kNorm, 20>(rs, x, lds, nrm, stream); return true;
        case 24: launch_partial<QT, kF32, kSegs, kNorm, 24>(rs, x, lds, nrm, stream); return true;
        case 38: launch_partial<QT, kF32, kSegs, kNorm, 38>(rs, x, lds, nrm, stream); return true;
        case 68:
            if constexpr (kNorm || 5 > QT::kMaxSteps) return false;
            else launch_partial<QT, kF32, kSegs, kNorm, 68>(rs, x, lds, nrm, stream);
            return true;
        case 100:
            if constexpr (kNorm || 7 > QT::kMaxSteps) return false;
            else launch_partial<QT, kF32, kSegs, kNorm, 100>(rs, x, lds, nrm, stream);
            return true;
        default: return false;
    }
}

// staged x (fp16 pairs), the x-sum table and 4 floats of reduction scratch
template <class QT>
size_t lds_bytes(int K) {
    return (size_t)K * 2 + (size_t)(K / kQK) * QT::kSxPerBlock * sizeof(float) + 4 * sizeof(float);
}

constexpr NormIn kNoNorm{nullptr, nullptr, nullptr, 0.f};

template <class QT, bool kF32>
hipError_t launch_matvec(const uint8_t* w, const uint16_t* x, void* y, int K, int N, hipStream_t stream) {
    const int nb = K / kQK;
    const size_t lds = lds_bytes<QT>(K);
    const RowSet rs{{w, w, w}, {y, y, y}, {N, N, N}};
    if (!launch_stream_for<QT, kF32, 1>(nb, rs, x, lds, kNoNorm, stream)) {
        // any other length: flat walk over the super-blocks of 4 rows
        constexpr int kRows = 4;
        // floor(f / nb) == (f * magic) >> 32 for every f < 2^20 (nb <= 112)
        const uint64_t magic = ((uint64_t)1 << 32) / (uint64_t)nb + 1u;
        const int rows_per_block = kRows * kWavesPerBlock;
        const int grid = (N + rows_per_block - 1) / rows_per_block;
        launch_kernel((matvec_flat_kernel<QT, kF32, kRows>), dim3(grid), dim3(kBlock), lds, stream, w, x, y, K,
                      N, magic);
    }
    return hipGetLastError();
}

template <class QT, bool kF32>
hipError_t launch_matvec_prologue(const uint8_t* w, const uint16_t* x, const NormIn& nrm, void* y, int K, int N,
                                  hipStream_t stream) {
    const RowSet rs{{w, w, w}, {y, y, y}, {N, N, N}};
    if (!launch_stream_for<QT, kF32, 1, true>(K / kQK, rs, x, lds_bytes<QT>(K), nrm, stream))
        return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int S, int M, bool kNorm, int NB = 0>
void launch_group_mixed(const RowSet& a, const RowSet& b, const uint16_t* x, int K, const NormIn& nrm,
                        hipStream_t stream) {
    // units of each set (Q4_K and Q6_K pack alike: four lanes per block)
    static_assert(Pack<Q4K, NB>::P == Pack<Q6K, NB>::P, "same packing");
    const int na = Pack<Q4K, NB>::units(a.end[2]), nbr = Pack<Q6K, NB>::units(b.end[2]);
    const size_t lds = std::max(lds_bytes<Q4K>(K), lds_bytes<Q6K>(K));
    if constexpr (S == 1) {
        if (na + nbr <= 8192) {
            // one pass, two rows per wave (attn_q/k/v at hidden 4096: measured
            // faster than streaming)
            constexpr int kM = 2;
            const int ga = (na + kM * kWavesPerBlock - 1) / (kM * kWavesPerBlock);
            const int gb = (nbr + kM * kWavesPerBlock - 1) / (kM * kWavesPerBlock);
            launch_kernel((matvec_group_kernel<Q4K, Q6K, 1, kM, false, kNorm, NB>), dim3(ga + gb), dim3(kBlock), lds,
                          stream, a, b, ga, x, K, nrm);
            return;
        }
    }
    // blocks split in proportion to the bytes each set streams
    const double ba = (double)na * Q4K::kBytes, bb = (double)nbr * Q6K::kBytes;
    const int grid = stream_grid(na + nbr);
    int ga = (int)(grid * ba / (ba + bb) + 0.5);
    ga = std::max(1, std::min(ga, std::min(grid - 1, stream_grid(na))));
    const int gb = std::max(1, std::min(grid - ga, stream_grid(nbr)));
    launch_kernel((matvec_group_kernel<Q4K, Q6K, S, M, true, kNorm, NB>), dim3(ga + gb), dim3(kBlock), lds, stream,
                  a, b, ga, x, K, nrm);
}

template <bool kNorm>
bool launch_group(int nb, RowSet (&set)[2], const int (&cnt)[2], bool f16, const uint16_t* x, int K,
                  const NormIn& nrm, hipStream_t s) {
    if (f16) return launch_stream_for<F16, false, 3, kNorm>(nb, set[0], x, lds_bytes<F16>(K), nrm, s);
    if (cnt[1] == 0) return launch_stream_for<Q4K, false, 3, kNorm>(nb, set[0], x, lds_bytes<Q4K>(K), nrm, s);
    if (cnt[0] == 0) return launch_stream_for<Q6K, false, 3, kNorm>(nb, set[1], x, lds_bytes<Q6K>(K), nrm, s);
    switch (nb) {
        case 16: launch_group_mixed<1, 1, kNorm>(set[0], set[1], x, K, nrm, s); return true;
        case 32: launch_group_mixed<2, 1, kNorm>(set[0], set[1], x, K, nrm, s); return true;
        case 48: launch_group_mixed<3, 1, kNorm>(set[0], set[1], x, K, nrm, s); return true;
        case 64: launch_group_mixed<4, 1, kNorm>(set[0], set[1], x, K, nrm, s); return true;
        case 4: launch_group_mixed<1, 1, kNorm, 4>(set[0], set[1], x, K, nrm, s); return true;
        case 8: launch_group_mixed<1, 1, kNorm, 8>(set[0], set[1], x, K, nrm, s); return true;
        case 10: launch_group_mixed<1, 1, kNorm, 10>(set[0], set[1], x, K, nrm, s); return true;
        case 12: launch_group_mixed<1, 1, kNorm, 12>(set[0], set[1], x, K, nrm, s); return true;
        case 20: launch_group_mixed<2, 1, kNorm, 20>(set[0], set[1], x, K, nrm, s); return true;
        case 24: launch_group_mixed<2, 1, kNorm, 24>(set[0], set[1], x, K, nrm, s); return true;
        case 38: launch_group_mixed<3, 1, kNorm, 38>(set[0], set[1], x, K, nrm, s); return true;
        default: return false;
    }
}

template <class QT, bool kNorm>
hipError_t launch_gate_up_t(const uint8_t* wg, const uint8_t* wu, const uint16_t* x, uint16_t* act, int K, int N,
                          const NormIn& nrm, hipStream_t stream) {
    const size_t lds = lds_bytes<QT>(K) + sizeof(int);   // + the unit counter
    int grid = device_cus();
    const int nb = K / kQK;
    const int per_unit = pack_rows(nb, QT::kSbPerStep);
    const int units = (N + per_unit - 1) / per_unit;
    const int need = (units + kGateUpWaves - 1) / kGateUpWaves;
    if (grid > need) grid = need;
    const dim3 g(grid), b(kGateUpBlock);
    switch (K / kQK) {
        case 16: launch_kernel((matvec_gate_up_kernel<QT, 1, kNorm>), g, b, lds, stream, wg, wu, x, act, K, N, nrm); break;
        case 32: launch_kernel((matvec_gate_up_kernel<QT, 2, kNorm>), g, b, lds, stream, wg, wu, x, act, K, N, nrm); break;
        // rows shorter than one wave step (Qwen3-0.6B: hidden 1024; 1.7B: 2048;
        // 4B: 2560), and hidden 5120 (Qwen3-14B / 32B)
        case 4: launch_kernel((matvec_gate_up_kernel<QT, 1, kNorm, 4>), g, b, lds, stream, wg, wu, x, act, K, N, nrm); break;
        case 8: launch_kernel((matvec_gate_up_kernel<QT, 1, kNorm, 8>), g, b, lds, stream, wg, wu, x, act, K, N, nrm); break;
        case 12: launch_kernel((matvec_gate_up_kernel<QT, 1, kNorm, 12>), g, b, lds, stream, wg, wu, x, act, K, N, nrm); break;
        case 10: launch_kernel((matvec_gate_up_kernel<QT, 1, kNorm, 10>), g, b, lds, stream, wg, wu, x, act, K, N, nrm); break;
        case 20: launch_kernel((matvec_gate_up_kernel<QT, 2, kNorm, 20>), g, b, lds, stream, wg, wu, x, act, K, N, nrm); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool kNorm>
hipError_t launch_gate_up(int kind, const uint8_t* wg, const uint8_t* wu, const uint16_t* x, uint16_t* act, int K,
                          int N, const NormIn& nrm, hipStream_t s) {
    switch (kind) {
        case 6: return launch_gate_up_t<Q6K, kNorm>(wg, wu, x, act, K, N, nrm, s);
        case 1: return launch_gate_up_t<F16, kNorm>(wg, wu, x, act, K, N, nrm, s);
        default: return launch_gate_up_t<Q4K, kNorm>(wg, wu, x, act, K, N, nrm, s);
    }
}

}  // namespace

bool matvec_fused_length(int K, bool norm) {
    if (K <= 0 || K % kQK != 0) return false;
    switch (K / kQK) {
        case 4: case 8: case 10: case 12: case 16: case 20: case 24: case 32: case 38: case 48: case 64: return true;
        case 68: case 100: return !norm;
        default: return false;
    }
}

bool matvec_gate_up_length(int K) {
    return K == 1024 || K == 2048 || K == 2560 || K == 3072 || K == 4096 || K == 5120 || K == 8192;
}

size_t matvec_lds_bytes(int kind, int K) {
    return kind == 6 ? lds_bytes<Q6K>(K) : kind == 1 ? lds_bytes<F16>(K) : lds_bytes<Q4K>(K);
}

hipError_t launch_matvec_f16_blocks(const uint16_t* w, const uint16_t* x, void* y, bool f32_out, int K, int N,
                                    hipStream_t s) {
    const uint8_t* wb = reinterpret_cast<const uint8_t*>(w);
    return f32_out ? launch_matvec<F16, true>(wb, x, y, K, N, s) : launch_matvec<F16, false>(wb, x, y, K, N, s);
}

hipError_t launch_matvec_q4k(const uint8_t* w, const uint16_t* x, void* y, bool f32_out, int K, int N,
                             hipStream_t s) {
    return f32_out ? launch_matvec<Q4K, true>(w, x, y, K, N, s) : launch_matvec<Q4K, false>(w, x, y, K, N, s);
}

hipError_t launch_matvec_q6k(const uint8_t* w, const uint16_t* x, void* y, bool f32_out, int K, int N,
                             hipStream_t s) {
    return f32_out ? launch_matvec<Q6K, true>(w, x, y, K, N, s) : launch_matvec<Q6K, false>(w, x, y, K, N, s);
}

hipError_t launch_matvec_norm(int kind, const uint8_t* w, const uint16_t* x, const NormIn& norm, void* y,
                              bool f32_out, int K, int N, hipStream_t s) {
    if (kind == 1)
        return f32_out ? launch_matvec_prologue<F16, true>(w, x, norm, y, K, N, s)
                       : launch_matvec_prologue<F16, false>(w, x, norm, y, K, N, s);
    if (kind == 6)
        return f32_out ? launch_matvec_prologue<Q6K, true>(w, x, norm, y, K, N, s)
                       : launch_matvec_prologue<Q6K, false>(w, x, norm, y, K, N, s);
    return f32_out ? launch_matvec_prologue<Q4K, true>(w, x, norm, y, K, N, s)
                   : launch_matvec_prologue<Q4K, false>(w, x, norm, y, K, N, s);
}

// count matrices (1..3) reading x: kinds[i] 4 = Q4_K, 6 = Q6_K, 1 = fp16
// (all or none), n[i] rows, fp16 outputs y[i].  hipErrorInvalidValue,
// nothing launched, for a length other than 1024, 2048, 3072, 4096, 8192,
// 12288 or 16384 or fp16 mixed with quantized matrices.
hipError_t launch_matvec_group(int count, const int* kinds, const uint8_t* const* w, const uint16_t* x,
                               uint16_t* const* y, const int* n, int K, const NormIn* norm, hipStream_t s) {
    RowSet set[2];
    int cnt[2] = {0, 0};
    int f16 = 0;
    for (int i = 0; i < count; ++i) f16 += kinds[i] == 1;
    if (f16 != 0 && f16 != count) return hipErrorInvalidValue;
    for (int i = 0; i < count; ++i) {
        const int t = kinds[i] == 6;
        const int j = cnt[t]++;
        set[t].w[j] = w[i];
        set[t].y[j] = y[i];
        set[t].end[j] = (j ? set[t].end[j - 1] : 0) + n[i];
    }
    for (int t = 0; t < 2; ++t)
        for (int j = cnt[t]; j < 3 && cnt[t] > 0; ++j) {
            set[t].w[j] = set[t].w[j - 1];
            set[t].y[j] = set[t].y[j - 1];
            set[t].end[j] = set[t].end[j - 1];
        }
    const int nb = K / kQK;
    const bool ok = norm ? launch_group<true>(nb, set, cnt, f16 != 0, x, K, *norm, s)
                         : launch_group<false>(nb, set, cnt, f16 != 0, x, K, kNoNorm, s);
    return ok ? hipGetLastError() : hipErrorInvalidValue;
}

// kind 4: Q4_K, 6: Q6_K, 1: fp16; in_features 1024, 2048, 3072, 4096 or
// 8192 (4, 8, 12, 16 or 32 blocks of 256)
hipError_t launch_matvec_gate_up_swiglu(int kind, const uint8_t* wg, const uint8_t* wu, const uint16_t* x,
                                        uint16_t* act, int K, int N, const NormIn* norm, hipStream_t s) {
    return norm ? launch_gate_up<true>(kind, wg, wu, x, act, K, N, *norm, s)
                : launch_gate_up<false>(kind, wg, wu, x, act, K, N, kNoNorm, s);
}

}  // namespace citlali::hip
