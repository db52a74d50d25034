// attention.hip -- single-token decode attention over the per-layer fp16 KV
// cache, split across workgroups (flash-decoding).
//
// Semantics follow kernels.cu:545-649 of the reference: for query head h
// (kv head h / (heads/kv_heads)) and cached positions t = 0..position,
// s_t = (q_h . K[t]) / sqrt(head_dim); p = softmax(s); out_h = sum_t p_t V[t],
// fp32 arithmetic, fp16 output rounded nearest-even.  Cache layout is the
// reference's [position][kv_head][head_dim] (kernels.cu:524-533).
//
// gfx950 design
//  * One workgroup (4 waves) per (position chunk, kv head, sequence); it
//    serves every query head of the GQA group, so K and V are read from HBM
//    once per kv head (the reference re-reads them per query head).
//  * Each wave streams tiles of positions: coalesced 128-bit loads of the K
//    and V rows into registers, staged through a wave-private LDS tile, with
//    the next tile's loads issued before the current tile is consumed.
//  * Scores: lane = (position, head); q of the lane's head lives in VGPRs as
//    fp16 pairs and v_dot2_f32_f16 accumulates in fp32.  The running max and
//    sum of the online softmax are butterflies over the lanes of one head.
//    Exponentials are taken in base 2 with log2(e) folded into the scale.
//  * Values: lane = (position group, 8-dim slice) accumulating every head of
//    the group, so each staged V row is read from LDS once per lane group;
//    p * V accumulates in fp32 and the groups are summed in the final merge.
//  * The four waves merge in LDS; a chunk writes (max, sum, acc[head_dim])
//    per head and a second kernel merges the chunks of each query head by
//    log-sum-exp.  A sequence that fits one chunk is written directly.
//    (Merging in the last workgroup of the same launch measured slower on
//    gfx950: the hand-off across XCDs needs write-through stores and an L2
//    invalidate.)
#include "device_common.hpp"
#include "launch.hpp"

#include <math.h>

#include <type_traits>

namespace citlali::hip {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxSplits = 512;   // plan_attention never makes more chunks

template <int HD, int GP>
struct Cfg {
    static_assert(HD == 64 || HD == 128, "head_dim");
    static_assert(GP == 1 || GP == 2 || GP == 4 || GP == 8, "group");
    static constexpr int kChunks = HD / 8;                 // 16-byte slices per row
    static constexpr int kTP = (64 / GP) < 32 ? 64 / GP : 32;   // positions per tile
    static constexpr int kStride = HD + 8;                 // padded LDS row (halves)
    static constexpr int kRowsPerLoad = kWave / kChunks;
    static constexpr int kLoads = kTP / kRowsPerLoad;      // per tile, for K and for V
    // value phase: lane = (position group, 8-dim slice), every head of the group
    static constexpr int kVGroups = kWave / kChunks;
    static constexpr int kVPerLane = kTP / kVGroups;       // positions per lane per tile
    static constexpr int kTileHalves = kTP * kStride;
    // wave-private region: K tile, V tile, p[kTP][GP], alpha[GP]; 16-byte multiple
    static constexpr size_t kWaveLds =
        (((size_t)kTileHalves * 2 * 2 + (size_t)GP * kTP * 4 + (size_t)GP * 4) + 15) & ~(size_t)15;
    // workgroup merge: (max, sum)[kWaves][GP], then acc[kWaves * kVGroups][GP][HD]
    static constexpr size_t kMlFloats = ((size_t)kWaves * GP * 2 + 3) & ~(size_t)3;
    static constexpr size_t kMergeLds = (kMlFloats + (size_t)kWaves * kVGroups * GP * HD) * sizeof(float);
    static_assert(kLoads >= 1 && kVPerLane >= 1 && kTP % kVGroups == 0, "tile");
};

template <int HD, int GP>
size_t split_lds_bytes() {
    using C = Cfg<HD, GP>;
    const size_t tiles = C::kWaveLds * kWaves;
    return tiles > C::kMergeLds ? tiles : C::kMergeLds;
}

// Positions a sequence covers and its chunk count.  A position at or beyond
// the caller's bound `max_len` is cut there, so neither the cache reads nor
// the chunk index leave their buffers.
struct SeqSpan {
    int len, n_valid;
};
__device__ __forceinline__ SeqSpan seq_span(const int32_t* positions, int position, int seq, int chunk,
                                            int max_len) {
    int L = (positions ? positions[seq] : position) + 1;
    L = min(L, max_len);
    return {L, L > 0 ? (L + chunk - 1) / chunk : 0};
}

// Grid: (chunk, kv_head, seq).  `positions` (device, per sequence) or the
// scalar `position` gives the last cached position of each sequence.
template <int HD, int GP, int kDepth>
__global__ __launch_bounds__(kBlock) void attn_split_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    long long seq_stride, const int32_t* __restrict__ positions, int position, int max_len, int heads,
    int kv_heads, int group, int chunk, float scale_log2, float* __restrict__ part, int n_splits,
    uint16_t* __restrict__ out) {
    using C = Cfg<HD, GP>;
    extern __shared__ __align__(16) uint8_t smem[];

    const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const SeqSpan span = seq_span(positions, position, seq, chunk, max_len);
    const int L = span.len, n_valid = span.n_valid;
    const int b0 = split * chunk;
    if (b0 >= L) return;
    const int b1 = min(L, b0 + chunk);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    // the chunk's positions split over the four waves in whole tiles (a
    // short sequence's only chunk still occupies every wave)
    const int sub = (((b1 - b0 + kWaves - 1) / kWaves + C::kTP - 1) / C::kTP) * C::kTP;
    const int w0 = min(b1, b0 + wave * sub);
    const int w1 = min(b1, w0 + sub);

    uint8_t* wl = smem + (size_t)wave * C::kWaveLds;
    uint16_t* kt = reinterpret_cast<uint16_t*>(wl);
    uint16_t* vt = kt + C::kTileHalves;
    float* pt = reinterpret_cast<float*>(vt + C::kTileHalves);   // [kTP][GP]
    float* at = pt + GP * C::kTP;                                 // [GP]

    const uint16_t* kbase = k_cache + (size_t)seq * seq_stride + (size_t)kvh * HD;
    const uint16_t* vbase = v_cache + (size_t)seq * seq_stride + (size_t)kvh * HD;
    const size_t row_step = (size_t)kv_heads * HD;

    // scores-phase identity
    const int sh = lane % GP, sp = lane / GP;
    const bool s_head_ok = sh < group;
    const bool s_lane_ok = sp < C::kTP;
    // q of the lane's head in VGPRs.  Unconditional loads (a padding head
    // reads the group's last head and is zeroed) keep every global load
    // outside branches, so the compiler's load counting stays exact and the
    // waits below never cover the tiles still in flight.
    uint32_t qv[HD / 2];
    {
        const int hq = kvh * group + (s_head_ok ? sh : group - 1);
        const uint16_t* qh = q + ((size_t)seq * heads + hq) * HD;
        const uint32_t keep = s_head_ok ? 0xffffffffu : 0u;
#pragma unroll
        for (int c = 0; c < C::kChunks; ++c) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(qh + c * 8);
            qv[4 * c + 0] = v.x & keep; qv[4 * c + 1] = v.y & keep;
            qv[4 * c + 2] = v.z & keep; qv[4 * c + 3] = v.w & keep;
        }
    }
    // value-phase identity: lane = (position group vg, 8-dim slice vc)
    const int vc = lane % C::kChunks, vg = lane / C::kChunks;
    float acc[GP][8];
#pragma unroll
    for (int h = 0; h < GP; ++h)
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[h][k] = 0.f;

    float m_run = -INFINITY, l_run = 0.f;   // per scores lane (head sh)

    // load identity; kDepth tiles of K and V rows in flight per wave
    const int lrow = lane / C::kChunks, lc = lane % C::kChunks;
    u32x4 kr[kDepth][C::kLoads], vr[kDepth][C::kLoads];
    auto load_tile = [&](u32x4 (&kd)[C::kLoads], u32x4 (&vd)[C::kLoads], int t0) {
#pragma unroll
        for (int i = 0; i < C::kLoads; ++i) {
            // branch-free: rows past the range re-read the last one (never used)
            const int pos = min(t0 + i * C::kRowsPerLoad + lrow, w1 - 1);
            kd[i] = *reinterpret_cast<const u32x4*>(kbase + (size_t)pos * row_step + lc * 8);
            vd[i] = *reinterpret_cast<const u32x4*>(vbase + (size_t)pos * row_step + lc * 8);
        }
    };

    // One staged tile; with nv <= 0 it changes nothing (scores -inf, weights 0).
    auto process_tile = [&](int t0) {
        const int nv = min(C::kTP, w1 - t0);

        // ---- scores + online softmax (lane = position sp, head sh) ----
        float s2 = -INFINITY;
        if (s_lane_ok && s_head_ok && sp < nv) {
            const uint16_t* kr_row = kt + sp * C::kStride;
            float a0 = 0.f, a1 = 0.f;
#pragma unroll
            for (int c = 0; c < C::kChunks; ++c) {
                const u32x4 kk = *reinterpret_cast<const u32x4*>(kr_row + c * 8);
                a0 = dot2(qv[4 * c + 0], kk.x, a0);
                a1 = dot2(qv[4 * c + 1], kk.y, a1);
                a0 = dot2(qv[4 * c + 2], kk.z, a0);
                a1 = dot2(qv[4 * c + 3], kk.w, a1);
            }
            s2 = (a0 + a1) * scale_log2;
        }
        const float mt = column_max<GP>(s2);
        const float m_new = fmaxf(m_run, mt);
        const bool live = m_new != -INFINITY;
        const float alpha = live ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
        const float pw = live ? __builtin_amdgcn_exp2f(s2 - m_new) : 0.f;
        const float ps = column_sum<GP>(pw);
        l_run = l_run * alpha + ps;
        m_run = m_new;
        if (s_lane_ok) pt[lane] = pw;   // lane = sp * GP + sh
        if (sp == 0) at[sh] = alpha;
        wave_lds_sync();

        // ---- values: every head for kVPerLane positions of this lane ----
        float al[GP];
        load_floats<GP>(at, al);
#pragma unroll
        for (int h = 0; h < GP; ++h)
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[h][k] *= al[h];
        // rows past nv hold finite copies of a valid row and weight 0
#pragma unroll
        for (int j = 0; j < C::kVPerLane; ++j) {
            const int p = vg + j * C::kVGroups;
            const u32x4 vv = *reinterpret_cast<const u32x4*>(vt + p * C::kStride + vc * 8);
            float pp[GP];
            load_floats<GP>(pt + p * GP, pp);
            const float v8[8] = {h2f(vv.x & 0xffffu), h2f(vv.x >> 16), h2f(vv.y & 0xffffu), h2f(vv.y >> 16),
                                 h2f(vv.z & 0xffffu), h2f(vv.z >> 16), h2f(vv.w & 0xffffu), h2f(vv.w >> 16)};
#pragma unroll
            for (int h = 0; h < GP; ++h)
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[h][k] = fmaf(pp[h], v8[k], acc[h][k]);
        }
        wave_lds_sync();
    };

    // kDepth tiles in flight: tile t is consumed while tiles t+1 .. t+kDepth-1
    // load, and its slot is refilled with tile t+kDepth right away.  Loads
    // are unconditional (past the range they re-read row w1 - 1, in bounds
    // even for an empty range since w1 = b1 >= 1 there) and a tile past the
    // range is a no-op, so no load sits in a branch.
    // The issue order is pinned (sched_barrier): the slots must be issued in
    // the same order as the loop refills them, or the wait before a slot's
    // first use covers the later slots too.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        load_tile(kr[d], vr[d], w0 + d * C::kTP);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int t0 = w0; t0 < w1; t0 += kDepth * C::kTP) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const int tt = t0 + d * C::kTP;
            // every row is stored: rows past the range hold a copy of row
            // w1 - 1 (finite) and get weight 0
#pragma unroll
            for (int i = 0; i < C::kLoads; ++i) {
                const int r = i * C::kRowsPerLoad + lrow;
                *reinterpret_cast<u32x4*>(kt + r * C::kStride + lc * 8) = kr[d][i];
                *reinterpret_cast<u32x4*>(vt + r * C::kStride + lc * 8) = vr[d][i];
            }
            wave_lds_sync();
            __builtin_amdgcn_sched_barrier(0);
            load_tile(kr[d], vr[d], tt + kDepth * C::kTP);
            __builtin_amdgcn_sched_barrier(0);
            process_tile(tt);
        }
    }

    // ---- merge the position groups and the four waves in LDS ----
    __syncthreads();   // every wave is done with its tiles
    float* ml = reinterpret_cast<float*>(smem);   // [kWaves][GP] (max, sum)
    float* ms = ml + C::kMlFloats;                // [kWaves * kVGroups][GP][HD]
    if (sp == 0) {
        ml[(wave * GP + sh) * 2] = m_run;
        ml[(wave * GP + sh) * 2 + 1] = l_run;
    }
#pragma unroll
    for (int h = 0; h < GP; ++h) {
        f32x4* e = reinterpret_cast<f32x4*>(ms + ((size_t)(wave * C::kVGroups + vg) * GP + h) * HD + vc * 8);
        e[0] = f32x4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
        e[1] = f32x4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
    }
    __syncthreads();

    for (int idx = threadIdx.x; idx < group * HD; idx += kBlock) {
        const int h = idx / HD, d = idx - h * HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, ml[(w * GP + h) * 2]);
        float Ls = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = ml[(w * GP + h) * 2];
            const float f = mw == -INFINITY ? 0.f : exp2f(mw - M);
            Ls += ml[(w * GP + h) * 2 + 1] * f;
            float a = 0.f;
#pragma unroll
            for (int g = 0; g < C::kVGroups; ++g) a += ms[((size_t)(w * C::kVGroups + g) * GP + h) * HD + d];
            A += a * f;
        }
        const int hq = kvh * group + h;
        if (n_valid == 1) {
            out[((size_t)seq * heads + hq) * HD + d] = f2h_rne(A / Ls);
        } else {
            float* pe = part + (((size_t)seq * heads + hq) * n_splits + split) * (HD + 4);
            pe[d] = A;
            if (d == 0) {
                pe[HD] = M;
                pe[HD + 1] = Ls;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// head_dim 128, GQA group 2..8: the same chunk / merge structure with both
// products on the matrix cores (v_mfma_f32_16x16x16f16).  The group's heads
// are the 16 MFMA columns (padding heads have q = 0 and are never written).
// Per wave, a tile of 16 positions, one tile's loads in flight:
//  * loads, two forms (kRows, chosen by the plan):
//    - direct: lane = (row col, 64-byte slab grp), 16 rows x 64 bytes per
//      instruction, K straight into the A operand, V into an LDS tile; the
//      refill is issued once the scores are in;
//    - rows (launches of more than two workgroups per CU, where HBM
//      saturates): each nontemporal instruction reads four whole 256-byte
//      rows (lane = row 4u + grp, 16-byte slice col), which a probe of the
//      same shape reads at ~7 TB/s against ~5.9 for 16 rows x 64 bytes;
//      K and V go to wave-private LDS rows, the refill is issued at once
//      and K is read back in the A operand layout.
//  * scores S[pos][head] = K[pos][:] . q[head][:]: the A operand is K row
//    `col` (lane = row `col`, a 64-byte slab `grp` of it; the 128
//    dims in 8 steps of 16, dim 32t + 8grp + 4h + j of step (t, h) being
//    operand k = 4grp + j), q is the B operand in the same dim order; lane
//    (col, grp) gets the scores of positions 4grp + i for head col.
//  * online softmax per head column (max and sum over the column's four lane
//    groups by permlane swaps), exponentials in base 2 as the VALU kernel.
//  * out^T[dim][head] += V^T[dim][pos] P^T[pos][head]: the scores' lane
//    layout is the B operand P^T as it stands, so every accumulator of a
//    lane belongs to the lane's head column and the online-softmax rescale
//    needs no lane moves (none on a wave's first tile).  P goes in as
//    fp16 hi + lo halves (two MFMAs), so its fp32 value counts to about
//    2^-22.  V rows are staged in a wave-private LDS tile and gathered per
//    lane as 4 positions x 4 dims, the A operand (dims 64c + 4col + e feed
//    output block 4c + e, rows 4grp + i of which are dims 64c + 16grp + 4i + e).
// ---------------------------------------------------------------------------
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
constexpr int kMTile = 16;                     // positions per MFMA tile
constexpr int kMStride = 128 + 8;              // K / V tile row in LDS (halves)
constexpr size_t kMWaveLds = (size_t)kMTile * kMStride * 2;
// merge: (max, sum)[NW][8], acc[NW][8 blocks][8 heads][4 lane groups][4]
// tiles: per wave a V tile, and with row loads a K tile, kMWaveLds each
template <int NW, bool kRows>
struct MfmaLds {
    static constexpr size_t kMlFloats = (size_t)NW * 8 * 2;
    static constexpr size_t kMerge = (kMlFloats + (size_t)NW * 2 * 8 * 16 * 4) * sizeof(float);
    static constexpr size_t kTiles = (kRows ? 2 : 1) * kMWaveLds * NW;
    static constexpr size_t kBytes = kMerge > kTiles ? kMerge : kTiles;
    // with the q/k prologue: q' of up to 8 heads, then per wave k' and v of the step
    static constexpr size_t kQs = kBytes;
    static constexpr size_t kKv = kQs + 8 * 128 * 2;
    static constexpr size_t kPrepBytes = kKv + (size_t)NW * 2 * 128 * 2;
};

__device__ __forceinline__ f32x4 mfma16(half4 a, half4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half4 as_half4(uint32_t lo, uint32_t hi) {
    return __builtin_bit_cast(half4, u32x2{lo, hi});
}

// kPrep: the launch also does the step's q/k head RMSNorm + RoPE and KV
// store (QkPrep).  Every workgroup forms q' of its group's heads (one wave
// per head, the arithmetic of the standalone kernel) while its first tiles
// load; the one wave whose positions end at the step's position forms k',
// stores k' and v into the caches and puts them in place of the cache row it
// loaded for that position (all lanes that load the row, clamped duplicates
// included), so nothing reads the row before it is written.
// Occupancy: left alone, the compiler allocates 160-164 registers per lane
// (VGPRs + accumulation registers), three waves per SIMD.  The row-load form
// serves launches of many workgroups per CU and is asked for four waves (it
// fits in 124-128 VGPRs, no spill); the direct form runs at most two
// workgroups per CU and keeps the allocation it schedules best with.
template <int GP, bool kRows, int NW, bool kPrep>
__global__ __launch_bounds__(NW * kWave, kRows ? 4 : 1) void attn_mfma_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    long long seq_stride, const int32_t* __restrict__ positions, int position, int max_len, int heads,
    int kv_heads, int group, int chunk, float scale_log2, float* __restrict__ part, int n_splits,
    uint16_t* __restrict__ out, QkPrep prep) {
    constexpr int HD = 128;
    static_assert(GP >= 2 && GP <= 8, "group");
    extern __shared__ __align__(16) uint8_t smem[];

    const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const SeqSpan span = seq_span(positions, position, seq, chunk, max_len);
    const int L = span.len, n_valid = span.n_valid;
    const int b0 = split * chunk;
    if (b0 >= L) return;
    const int b1 = min(L, b0 + chunk);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int col = lane & 15, grp = lane >> 4;
    const int sub = (((b1 - b0 + NW - 1) / NW + kMTile - 1) / kMTile) * kMTile;
    const int w0 = min(b1, b0 + wave * sub);
    const int w1 = min(b1, w0 + sub);

    // the step's position (kPrep): within the planned range it is the last
    // position L - 1 and lies in exactly one wave's range
    const int p_raw = positions ? positions[seq] : position;
    const int pos_row = L - 1;
    const bool has_pos = kPrep && p_raw >= 0 && p_raw < max_len && w0 <= pos_row && pos_row < w1;

    using Lds = MfmaLds<NW, kRows>;
    uint16_t* vt = reinterpret_cast<uint16_t*>(smem + (size_t)wave * (kRows ? 2 : 1) * kMWaveLds);
    uint16_t* kt = vt + kMTile * kMStride;   // row loads only
    // direct: lane = (row col, 64-byte slab grp); rows: lane = (row 4u + grp,
    // 16-byte slice col of the kv head's 256-byte row)
    const int lane_off = kRows ? 8 * col : 8 * grp;
    const uint16_t* kbase = k_cache + (size_t)seq * seq_stride + (size_t)kvh * HD + lane_off;
    const uint16_t* vbase = v_cache + (size_t)seq * seq_stride + (size_t)kvh * HD + lane_off;
    const size_t row_step = (size_t)kv_heads * HD;

    // q of head `col` (zero past the group) as B operands, dims 32t + 8grp + 4h
    // + j; loaded here, turned into operands after the first tiles' loads are
    // issued, so that q's round trip overlaps theirs
    const bool q_ok = col < group;
    u32x4 q_raw[4];
    // kPrep: raw q of the heads this wave forms (dims lane, lane + 64), the
    // step's k and v of this kv head, the norm weights; all loads
    // unconditional (a missing weight reads q and is not used)
    constexpr int kHeadsPerWave = (GP + NW - 1) / NW;
    uint16_t pq[kHeadsPerWave][2], pk[2], pv[2], pqw[2], pkw[2];
    if constexpr (kPrep) {
#pragma unroll
        for (int j = 0; j < kHeadsPerWave; ++j) {
            const int h = min(wave + j * NW, group - 1);
            const uint16_t* qh = q + ((size_t)seq * heads + kvh * group + h) * HD;
            pq[j][0] = qh[lane];
            pq[j][1] = qh[64 + lane];
        }
        const size_t kv_off = ((size_t)seq * kv_heads + kvh) * HD;
        const uint16_t* qw = prep.q_norm ? prep.q_norm : q;
        const uint16_t* kw = prep.k_norm ? prep.k_norm : q;
        pk[0] = prep.k[kv_off + lane];
        pk[1] = prep.k[kv_off + 64 + lane];
        pv[0] = prep.v[kv_off + lane];
        pv[1] = prep.v[kv_off + 64 + lane];
        pqw[0] = qw[lane];
        pqw[1] = qw[64 + lane];
        pkw[0] = kw[lane];
        pkw[1] = kw[64 + lane];
    } else {
        const uint16_t* qh = q + ((size_t)seq * heads + kvh * group + (q_ok ? col : group - 1)) * HD + 8 * grp;
#pragma unroll
        for (int t = 0; t < 4; ++t) q_raw[t] = *reinterpret_cast<const u32x4*>(qh + 32 * t);
    }
    half4 qb[4][2];
    f32x4 o[8];   // o[4c + e][i]: dim 64c + 16grp + 4i + e of head col
#pragma unroll
    for (int b = 0; b < 8; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;   // head col

    // One tile of K and V rows in flight; branch-free (rows past the range
    // re-read row w1 - 1, in bounds also for an empty range).  Slot u of a
    // lane: direct, row t0 + col, dims 32u + 8grp .. + 7; rows, row
    // t0 + 4u + grp, dims 8col .. + 7.
    u32x4 kr[4], vr[4];
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if constexpr (kRows) {
                const size_t pos = (size_t)min(t0 + 4 * u + grp, w1 - 1);
                kr[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kbase + pos * row_step));
                vr[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vbase + pos * row_step));
            } else {
                const size_t pos = (size_t)min(t0 + col, w1 - 1);
                kr[u] = *reinterpret_cast<const u32x4*>(kbase + pos * row_step + 32 * u);
                vr[u] = *reinterpret_cast<const u32x4*>(vbase + pos * row_step + 32 * u);
            }
        }
    };

    const uint16_t* kv_new = reinterpret_cast<const uint16_t*>(smem + Lds::kKv) + (size_t)wave * 2 * HD;
    auto process = [&](int t0, auto first_tile) {
        if constexpr (kPrep) {
            // the step's row comes from the prologue's k' and v in LDS
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int row = kRows ? t0 + 4 * u + grp : t0 + col;
                if (has_pos && min(row, w1 - 1) == pos_row) {
                    const int dim = kRows ? 8 * col : 32 * u + 8 * grp;
                    kr[u] = *reinterpret_cast<const u32x4*>(kv_new + dim);
                    vr[u] = *reinterpret_cast<const u32x4*>(kv_new + HD + dim);
                }
            }
        }
        f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (kRows) {
            // both tiles into LDS rows; the slot is then free: refill it with
            // the next tile, in flight over this tile's whole computation
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                *reinterpret_cast<u32x4*>(vt + (4 * u + grp) * kMStride + 8 * col) = vr[u];
                *reinterpret_cast<u32x4*>(kt + (4 * u + grp) * kMStride + 8 * col) = kr[u];
            }
            __builtin_amdgcn_sched_barrier(0);
            load_tile(t0 + kMTile);
            __builtin_amdgcn_sched_barrier(0);
            wave_lds_sync();   // the K and V rows stored above
            // K row col, dims 32t + 8grp .. + 7: the A operand layout
            u32x4 kk[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) kk[t] = *reinterpret_cast<const u32x4*>(kt + col * kMStride + 32 * t + 8 * grp);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s = mfma16(as_half4(kk[t].x, kk[t].y), qb[t][0], s);
                s = mfma16(as_half4(kk[t].z, kk[t].w), qb[t][1], s);
            }
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) *reinterpret_cast<u32x4*>(vt + col * kMStride + 32 * t + 8 * grp) = vr[t];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s = mfma16(as_half4(kr[t].x, kr[t].y), qb[t][0], s);
                s = mfma16(as_half4(kr[t].z, kr[t].w), qb[t][1], s);
            }
            // the slot is consumed: refill it with the next tile (the address
            // waits for the scores, so the load is issued after them)
            load_tile(issue_after(t0 + kMTile, s[0], s[3]));
            __builtin_amdgcn_sched_barrier(0);
        }

        float sv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = t0 + 4 * grp + i < w1 ? s[i] * scale_log2 : -INFINITY;
        const float mt = column_max<16>(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
        const float m_new = fmaxf(m_run, mt);
        const bool live = m_new != -INFINITY;
        const float alpha = live ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
        float pv[4];
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pv[i] = live ? __builtin_amdgcn_exp2f(sv[i] - m_new) : 0.f;
            ps += pv[i];
        }
        l_run = l_run * alpha + column_sum<16>(ps);
        m_run = m_new;

        // rescale this lane's head (column col); not on the wave's first tile,
        // where o is still zero.  The decode launch (kPrep: one or two tiles
        // per wave) also skips it when no column's max moved; in the launches
        // of longer ranges that branch inside the loop measured slower
        // (config 3: 14.5 against 13.8 us), so they peel the first tile.
        if constexpr (kPrep) {
            if (t0 != w0 && __builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
#pragma unroll
                for (int b = 0; b < 8; ++b) o[b] *= alpha;
            }
        } else if constexpr (!decltype(first_tile)::value) {
#pragma unroll
            for (int b = 0; b < 8; ++b) o[b] *= alpha;
        }
        half4 ph, pl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const _Float16 h = (_Float16)pv[j];
            ph[j] = h;
            pl[j] = (_Float16)(pv[j] - (float)h);
        }
        if constexpr (!kRows) wave_lds_sync();   // the V rows stored above
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            uint32_t w[4][2];   // rows 4grp + j, dims 64c + 4col .. + 3
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x2 x = *reinterpret_cast<const u32x2*>(vt + (4 * grp + j) * kMStride + 64 * c + 4 * col);
                w[j][0] = x.x;
                w[j][1] = x.y;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
                const half4 vb = as_half4(__builtin_amdgcn_perm(w[1][e >> 1], w[0][e >> 1], sel),
                                          __builtin_amdgcn_perm(w[3][e >> 1], w[2][e >> 1], sel));
                // V^T P^T: dims x heads, so a lane's accumulators belong to
                // one head (its column) and the rescale needs no lane moves
                o[4 * c + e] = mfma16(vb, ph, o[4 * c + e]);
                o[4 * c + e] = mfma16(vb, pl, o[4 * c + e]);
            }
        }
        wave_lds_sync();   // before the next tile overwrites the rows
    };

    __builtin_amdgcn_sched_barrier(0);
    load_tile(w0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kPrep) {
        uint16_t* qs = reinterpret_cast<uint16_t*>(smem + Lds::kQs);   // [GP][HD]
        // the RoPE angle of this lane's dim pair at the step's position: the
        // same for every head, and independent of the loads in flight
        float rsn, rcs;
        rope_angle(lane, HD, p_raw, prep.theta, rsn, rcs);
#pragma unroll
        for (int j = 0; j < kHeadsPerWave; ++j) {
            const int h = wave + j * NW;
            if (h < GP) {   // wave-uniform
                uint16_t y0 = pq[j][0], y1 = pq[j][1];
                if (prep.q_norm != nullptr) {
                    const float x0 = h2f(y0), x1 = h2f(y1);
                    const float inv = head_inv_rms(x0, x1, HD, prep.eps);
                    y0 = f2h_rne(x0 * inv * h2f(pqw[0]));
                    y1 = f2h_rne(x1 * inv * h2f(pqw[1]));
                }
                uint16_t r0, r1;
                rope_rotate(h2f(y0), h2f(y1), rsn, rcs, r0, r1);
                const bool real = h < group;   // padding heads: q = 0
                qs[h * HD + lane] = real ? r0 : (uint16_t)0;
                qs[h * HD + 64 + lane] = real ? r1 : (uint16_t)0;
            }
        }
        if (has_pos) {   // wave-uniform
            uint16_t y0 = pk[0], y1 = pk[1];
            if (prep.k_norm != nullptr) {
                const float x0 = h2f(y0), x1 = h2f(y1);
                const float inv = head_inv_rms(x0, x1, HD, prep.eps);
                y0 = f2h_rne(x0 * inv * h2f(pkw[0]));
                y1 = f2h_rne(x1 * inv * h2f(pkw[1]));
            }
            uint16_t r0, r1;
            rope_rotate(h2f(y0), h2f(y1), rsn, rcs, r0, r1);
            const size_t row = (size_t)seq * seq_stride + (size_t)pos_row * row_step + (size_t)kvh * HD;
            prep.k_cache[row + lane] = r0;
            prep.k_cache[row + 64 + lane] = r1;
            prep.v_cache[row + lane] = pv[0];
            prep.v_cache[row + 64 + lane] = pv[1];
            uint16_t* kvw = reinterpret_cast<uint16_t*>(smem + Lds::kKv) + (size_t)wave * 2 * HD;
            kvw[lane] = r0;
            kvw[64 + lane] = r1;
            kvw[HD + lane] = pv[0];
            kvw[HD + 64 + lane] = pv[1];
        }
        lds_barrier();   // q' of every head, and this wave's k' / v (tile loads stay in flight)
        const uint16_t* qh = qs + (q_ok ? col : 0) * HD + 8 * grp;
        const uint32_t keep = q_ok ? 0xffffffffu : 0u;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(qh + 32 * t);
            qb[t][0] = as_half4(v.x & keep, v.y & keep);
            qb[t][1] = as_half4(v.z & keep, v.w & keep);
        }
    } else {
        const uint32_t keep = q_ok ? 0xffffffffu : 0u;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            qb[t][0] = as_half4(q_raw[t].x & keep, q_raw[t].y & keep);
            qb[t][1] = as_half4(q_raw[t].z & keep, q_raw[t].w & keep);
        }
    }
    if constexpr (kPrep) {
        for (int t0 = w0; t0 < w1; t0 += kMTile) process(t0, std::false_type{});
    } else {
        if (w0 < w1) process(w0, std::true_type{});
        for (int t0 = w0 + kMTile; t0 < w1; t0 += kMTile) process(t0, std::false_type{});
    }

    // ---- merge the waves in LDS ----
    __syncthreads();   // every wave is done with its V tile
    float* ml = reinterpret_cast<float*>(smem);   // [NW][8] (max, sum)
    float* ms = ml + Lds::kMlFloats;              // [NW][8 b][8 heads][4 grp][4 i]
    if (grp == 0 && col < GP) {
        ml[(wave * 8 + col) * 2] = m_run;
        ml[(wave * 8 + col) * 2 + 1] = l_run;
    }
    if (col < GP) {
#pragma unroll
        for (int b = 0; b < 8; ++b)
            *reinterpret_cast<f32x4*>(ms + ((((size_t)wave * 8 + b) * 8 + col) * 4 + grp) * 4) = o[b];
    }
    __syncthreads();

    // Thread t merges dims kPer*t .. + kPer - 1 of one head (kPer divides HD):
    // the head's max, wave factors and sum are formed once, and every LDS
    // read is issued before the arithmetic.
    constexpr int kPer = GP * HD / (NW * kWave);
    static_assert(kPer >= 1 && HD % kPer == 0 && kPer * NW * kWave == GP * HD, "merge split");
    const int base = (int)threadIdx.x * kPer;
    if (base >= group * HD) return;
    const int h = base / HD, dim0 = base - h * HD;
    f32x2 mlw[NW];
    float acc[NW][kPer];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        mlw[w] = *reinterpret_cast<const f32x2*>(ml + (w * 8 + h) * 2);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            // dim = 64c + 16g + 4i + e lives in o[4c + e][i] of lane group g
            const int dim = dim0 + j;
            const int b = 4 * (dim >> 6) + (dim & 3), g4 = (dim >> 4) & 3, i4 = (dim >> 2) & 3;
            acc[w][j] = ms[((((size_t)w * 8 + b) * 8 + h) * 4 + g4) * 4 + i4];
        }
    }
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, mlw[w].x);
    float Ls = 0.f, A[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) A[j] = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const float f = mlw[w].x == -INFINITY ? 0.f : exp2f(mlw[w].x - M);
        Ls += mlw[w].y * f;
#pragma unroll
        for (int j = 0; j < kPer; ++j) A[j] += acc[w][j] * f;
    }
    const int hq = kvh * group + h;
    if (n_valid == 1) {
        uint16_t* o = out + ((size_t)seq * heads + hq) * HD + dim0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) o[j] = f2h_rne(A[j] / Ls);
    } else {
        float* pe = part + (((size_t)seq * heads + hq) * n_splits + split) * (HD + 4);
#pragma unroll
        for (int j = 0; j < kPer; ++j) pe[dim0 + j] = A[j];
        if (dim0 == 0) {
            pe[HD] = M;
            pe[HD + 1] = Ls;
        }
    }
}

// Grid: (query head x dim part, seq).  Log-sum-exp merge of one head's chunk
// partials ([chunk][HD + 4]: acc[HD], max, sum) in one global round trip,
// without LDS: a workgroup owns HD / kParts dims of one head; every wave
// finds the largest chunk max M (lane j reads the maxima of chunks j,
// j + 64, ...) while thread (dim quad, subset g) loads the accumulators and
// (max, sum) of its chunks g, g + kSub, ...; it folds them with the factors
// exp2(max - M) in chunk order, and the kSub consecutive lanes of a dim quad
// add their folds by DPP.  More parts give more workgroups, each thread
// fewer chunks.
template <int HD, int kParts, int kBatch>
__global__ __launch_bounds__(kBlock) void attn_merge_kernel(const float* __restrict__ part,
                                                            const int32_t* __restrict__ positions, int position,
                                                            int max_len, int heads, int chunk, int n_splits,
                                                            uint16_t* __restrict__ out) {
    const int hq = blockIdx.x / kParts, dpart = blockIdx.x % kParts, seq = blockIdx.y;
    const int n_valid = seq_span(positions, position, seq, chunk, max_len).n_valid;
    if (n_valid <= 1) return;   // written by the split kernel
    const size_t h0 = (size_t)seq * heads + hq;
    constexpr size_t ent = HD + 4;
    const float* hp = part + h0 * n_splits * ent;
    constexpr int kQuads = HD / 4 / kParts;   // dim quads of this workgroup
    constexpr int kSub = kBlock / kQuads;     // lanes per dim quad
    static_assert(kSub == 8 || kSub == 16 || kSub == 32, "subsets of consecutive lanes");
    const int lane = threadIdx.x & (kWave - 1);
    const int g = threadIdx.x % kSub, d4 = dpart * kQuads + threadIdx.x / kSub;

    // kBatch chunks per thread have their loads issued together; the loads
    // are unconditional (a chunk past the last re-reads the last one), so
    // none waits on a branch, and such chunks get the factor 0.
    auto load_batch = [&](int s0, f32x4 (&v)[kBatch], f32x2 (&ml)[kBatch]) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const float* e = hp + (size_t)min(s0 + j * kSub, n_valid - 1) * ent;
            ml[j] = *reinterpret_cast<const f32x2*>(e + HD);
            v[j] = *reinterpret_cast<const f32x4*>(e + 4 * d4);
        }
    };
    f32x4 v[kBatch];
    f32x2 ml[kBatch];
    load_batch(g, v, ml);
    // the largest chunk max (its loads go out behind the first batch's)
    float mx = -INFINITY;
    for (int s = lane; s < kMaxSplits; s += kWave) {   // uniform trip count
        mx = fmaxf(mx, hp[(size_t)min(s, n_valid - 1) * ent + HD]);
        if (s - lane + kWave >= n_valid) break;
    }
    const float M = wave_max(mx);

    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
    for (int s0 = g;;) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const float mj = s0 + j * kSub < n_valid ? ml[j].x : -INFINITY;
            const float f = mj == -INFINITY ? 0.f : exp2f(mj - M);
            a += v[j] * f;
            l += ml[j].y * f;
        }
        s0 += kBatch * kSub;
        if (s0 - g >= n_valid) break;   // uniform: no chunk left for any subset
        load_batch(s0, v, ml);
    }
    a.x = lane_group_sum<kSub>(a.x);
    a.y = lane_group_sum<kSub>(a.y);
    a.z = lane_group_sum<kSub>(a.z);
    a.w = lane_group_sum<kSub>(a.w);
    l = lane_group_sum<kSub>(l);
    if (g == 0) {
        const float inv = 1.f / l;
        uint16_t* o = out + h0 * HD + 4 * d4;
        o[0] = f2h_rne(a.x * inv);
        o[1] = f2h_rne(a.y * inv);
        o[2] = f2h_rne(a.z * inv);
        o[3] = f2h_rne(a.w * inv);
    }
}

// The merge launch, its per-thread batch sized to the plan's chunk count.
template <int HD, int kParts>
void launch_merge_parts(const AttnArgs& a, const AttnPlan& p, hipStream_t stream) {
    constexpr int kSub = kBlock / (HD / 4 / kParts);
    const int per = (p.n_splits + kSub - 1) / kSub;
    auto go = [&](auto kernel) {
        // no LDS: the merge keeps everything in registers
        launch_kernel(kernel, dim3(a.heads * kParts, a.nseq), dim3(kBlock), 0, stream, a.workspace, a.positions,
                      a.position, a.max_len, a.heads, p.chunk, p.n_splits, a.out);
    };
    if (per <= 1) go(attn_merge_kernel<HD, kParts, 1>);
    else if (per <= 2) go(attn_merge_kernel<HD, kParts, 2>);
    else if (per <= 4) go(attn_merge_kernel<HD, kParts, 4>);
    else go(attn_merge_kernel<HD, kParts, 8>);
}

// Launches of fewer than kMergeSpreadBelow (head, sequence) pairs -- one
// sequence -- split each head's dims over up to four workgroups, so that a
// thread folds one chunk where the lanes allow (config 3, L = 8192, 32 chunks:
// 128 workgroups; config-5 lengths, 9-12 chunks: 64).  Measured on MI355X
// against one workgroup per head: split + merge 13.40 against 13.50 us at
// config 3, 6.29 against 6.38 us per attention at config-5 lengths in a
// graph; config 4 (16 sequences, 512 heads) measured 1-2% slower spread, so
// launches of many heads keep one workgroup per head.
constexpr int kMergeSpreadBelow = 256;
template <int HD>
void launch_merge(const AttnArgs& a, const AttnPlan& p, hipStream_t stream) {
    constexpr int kSub1 = kBlock / (HD / 4);   // lanes per dim quad with one part: 8 (HD 128), 16 (HD 64)
    if (a.heads * a.nseq >= kMergeSpreadBelow || p.n_splits <= kSub1) {
        launch_merge_parts<HD, 1>(a, p, stream);
    } else if constexpr (kSub1 * 4 <= 32) {
        if (p.n_splits <= 2 * kSub1) launch_merge_parts<HD, 2>(a, p, stream);
        else launch_merge_parts<HD, 4>(a, p, stream);
    } else {
        launch_merge_parts<HD, 2>(a, p, stream);
    }
}

template <int HD, int GP, int kDepth>
hipError_t launch_split(const AttnArgs& a, const AttnPlan& p, hipStream_t stream) {
    const size_t lds = split_lds_bytes<HD, GP>();
    const float scale_log2 = (float)(1.4426950408889634 / sqrt((double)HD));
    launch_kernel_in_call(p.n_splits <= 1, (attn_split_kernel<HD, GP, kDepth>), dim3(p.n_splits, a.kv_heads, a.nseq),
                          dim3(kBlock), lds, stream, a.q, a.k_cache, a.v_cache, a.seq_stride, a.positions,
                          a.position, a.max_len, a.heads, a.kv_heads, a.heads / a.kv_heads, p.chunk, scale_log2,
                          a.workspace, p.n_splits, a.out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.n_splits <= 1) return e;
    launch_merge<HD>(a, p, stream);
    return hipGetLastError();
}

template <int GP, bool kRows, int NW = kWaves>
hipError_t launch_mfma(const AttnArgs& a, const AttnPlan& p, hipStream_t stream) {
    const float scale_log2 = (float)(1.4426950408889634 / sqrt(128.0));
    const dim3 grid(p.n_splits, a.kv_heads, a.nseq);
    if (a.prep != nullptr) {
        launch_kernel_in_call(p.n_splits <= 1, (attn_mfma_kernel<GP, kRows, NW, true>), grid, dim3(NW * kWave),
                              MfmaLds<NW, kRows>::kPrepBytes, stream, a.q, a.k_cache, a.v_cache, a.seq_stride, a.positions,
                              a.position, a.max_len, a.heads, a.kv_heads, a.heads / a.kv_heads, p.chunk, scale_log2,
                              a.workspace, p.n_splits, a.out, *a.prep);
    } else {
        launch_kernel_in_call(p.n_splits <= 1, (attn_mfma_kernel<GP, kRows, NW, false>), grid, dim3(NW * kWave),
                              MfmaLds<NW, kRows>::kBytes, stream, a.q, a.k_cache, a.v_cache, a.seq_stride, a.positions,
                              a.position, a.max_len, a.heads, a.kv_heads, a.heads / a.kv_heads, p.chunk, scale_log2,
                              a.workspace, p.n_splits, a.out, QkPrep{});
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.n_splits <= 1) return e;
    launch_merge<128>(a, p, stream);
    return hipGetLastError();
}

template <int HD, int GP>
hipError_t launch_depth(const AttnArgs& a, const AttnPlan& p, hipStream_t s) {
    if constexpr (HD == 128 && GP >= 2) {
        // one tile in flight per wave; the plan picks the load form
        if (p.depth != 1) return hipErrorInvalidValue;
        return p.rows ? launch_mfma<GP, true>(a, p, s) : launch_mfma<GP, false>(a, p, s);
    }
    if (a.prep != nullptr) return hipErrorInvalidValue;   // the q/k prologue exists only in the MFMA kernel
    switch (p.depth) {
        case 1: return launch_split<HD, GP, 1>(a, p, s);
        case 2: return launch_split<HD, GP, 2>(a, p, s);
        default: return hipErrorInvalidValue;
    }
}

template <int HD>
hipError_t launch_hd(const AttnArgs& a, const AttnPlan& p, hipStream_t s) {
    switch (p.gp) {
        case 1: return launch_depth<HD, 1>(a, p, s);
        case 2: return launch_depth<HD, 2>(a, p, s);
        case 4: return launch_depth<HD, 4>(a, p, s);
        case 8: return launch_depth<HD, 8>(a, p, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool attention_supported(int head_dim, int group) {
    return (head_dim == 64 || head_dim == 128) && group >= 1 && group <= 8;
}

int attention_plan_length(int length, int max_context) {
    long long b = 256;
    while (b < length) b <<= 1;
    return b < max_context ? (int)b : max_context;
}

// Work split: enough chunks for about `target_blocks` workgroups over all
// (sequence, kv head) units, within a range of chunk lengths that keeps the
// per-workgroup set-up and the partial write amortised -- for the
// matrix-core kernel (head_dim 128, group >= 2) 64 positions up to 1024 with
// at most 16 units, 512 with more; 256..512 for the other kernel (measured
// on MI355X: one sequence at 512..32768 positions, 16 sequences of
// 4096..32768); the chunk a multiple of 4 tiles, and at most kMaxSplits
// chunks (bounds the merge's per-thread loop and the partials workspace).
AttnPlan plan_attention(int max_len, int nseq, int kv_heads, int heads, int head_dim, int target_blocks) {
    AttnPlan p{};
    const int group = heads / kv_heads;
    p.gp = group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8;
    const bool mfma = head_dim == 128 && p.gp >= 2;
    const int tp = mfma ? kMTile : (64 / p.gp) < 32 ? 64 / p.gp : 32;
    const int quantum = tp * kWaves;
    const long long units = (long long)nseq * kv_heads;
    const long long lo = mfma ? 64 : 256, hi = mfma ? (units <= 16 ? 1024 : 512) : 512;
    long long chunk = ((long long)max_len * units + target_blocks - 1) / target_blocks;
    chunk = chunk < lo ? lo : chunk > hi ? hi : chunk;
    const long long min_chunk = ((long long)max_len + kMaxSplits - 1) / kMaxSplits;
    if (chunk < min_chunk) chunk = min_chunk;
    chunk = ((chunk + quantum - 1) / quantum) * quantum;
    p.chunk = (int)chunk;
    p.n_splits = (int)((max_len + chunk - 1) / chunk);
    // one tile in flight per wave: deeper rings measured no faster on
    // gfx950 (the per-tile work, not the load latency, bounds a wave)
    p.depth = 1;
    // whole-row loads once the launch holds more than two workgroups per CU
    // (HBM saturates; measured at config 4: 251 against 298-308 us), direct
    // loads below (latency-bound launches: 0.1-0.2 us faster)
    p.rows = mfma && units * p.n_splits > 2LL * target_blocks;
    return p;
}

size_t attention_workspace_bytes(const AttnPlan& p, int nseq, int heads, int head_dim) {
    if (p.n_splits <= 1) return 0;
    return (size_t)nseq * heads * p.n_splits * (head_dim + 4) * sizeof(float);
}

// The split count is not monotone in the planned length: the chunk is
// rounded up to whole tiles, so a longer plan can need fewer chunks (32/8
// heads: 2048 positions plan 32 chunks of 64, 3000 plan 24 of 128).  Every
// term of the chunk formula is non-decreasing in the length, so within a
// run of lengths sharing one chunk the count peaks at the run's last length;
// the walk visits those lengths only, from max_len down (a binary search
// finds where the next shorter chunk ends), a few dozen plans in all.
size_t attention_workspace_bound(int max_len, int nseq, int kv_heads, int heads, int head_dim, int target_blocks) {
    int most = 0;
    for (int len = max_len; len >= 1;) {
        const AttnPlan p = plan_attention(len, nseq, kv_heads, heads, head_dim, target_blocks);
        if (p.n_splits > most) most = p.n_splits;
        int lo = 0, hi = len - 1;   // the longest length with a shorter chunk, 0 if none
        while (lo < hi) {
            const int mid = lo + (hi - lo + 1) / 2;
            if (plan_attention(mid, nseq, kv_heads, heads, head_dim, target_blocks).chunk < p.chunk)
                lo = mid;
            else
                hi = mid - 1;
        }
        len = lo;
    }
    AttnPlan worst{};
    worst.n_splits = most;
    return attention_workspace_bytes(worst, nseq, heads, head_dim);
}

hipError_t launch_attention(const AttnArgs& a, const AttnPlan& p, hipStream_t s) {
    if (a.head_dim == 128) return launch_hd<128>(a, p, s);
    if (a.head_dim == 64) return launch_hd<64>(a, p, s);
    return hipErrorInvalidValue;
}

}  // namespace citlali::hip
