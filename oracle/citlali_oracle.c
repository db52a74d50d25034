/*
 * citlali_oracle.c -- CPU restatement of the Citlali decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see citlali_oracle.h): used by tests/, by
 * __graft_entry__.smoke() as the checker and by bench.py's cpu_baseline leg.
 * Never linked into or called by the product.
 *
 * Reference paths below are relative to the Citlali-LLM-Engine repository.
 */
#include "citlali_oracle.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static int pick_threads(int n) { return n > 0 ? n : orc_num_threads(); }

/* ------------------------------------------------------------------------ *
 * fp16 <-> fp32
 * ------------------------------------------------------------------------ */

/* dtype.cpp:136-176 (float_to_half_bits).  Round to nearest with ties away
 * from zero: the decision looks only at the most significant dropped bit.
 * Exponent overflow (including Inf and NaN inputs) gives signed infinity;
 * magnitudes below 2^-25 flush to signed zero (dtype.cpp:146-148). */
uint16_t orc_f2h(float v) {
    const uint32_t u = f2u(v);
    const uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
    const int e16 = (int)((u >> 23) & 0xffu) - 112;   /* rebias 127 -> 15 */
    const uint32_t frac = u & 0x7fffffu;
    if (e16 >= 31) return (uint16_t)(s | 0x7c00u);
    if (e16 > 0) {
        uint32_t h = ((uint32_t)e16 << 10) | (frac >> 13);
        h += (frac >> 12) & 1u;             /* carry may ripple into the exponent */
        return (uint16_t)(s | h);
    }
    if (e16 < -10) return s;
    /* fp16 subnormal: significand with hidden bit, shifted right by 14 - e16 */
    const uint32_t sig = frac | 0x800000u;
    const unsigned sh = (unsigned)(14 - e16);   /* 14..24 */
    uint32_t h = sig >> sh;
    h += (sig >> (sh - 1)) & 1u;
    return (uint16_t)(s | h);
}

/* dtype.cpp:76-133 (half_bits_to_float): exact widening; Inf/NaN keep their
 * payload bits shifted into the fp32 fraction. */
float orc_h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
    float mag = (e == 0) ? ldexpf((float)m, -24) : ldexpf((float)(m | 0x400u), (int)e - 25);
    return s ? -mag : mag;
}

/* IEEE binary16 round-to-nearest-even (the rule of the device conversion
 * __float2half used by store_half, kernels.cu:21-24).  NaN -> quiet NaN. */
uint16_t orc_f2h_rne(float v) {
    const uint32_t u = f2u(v);
    const uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t ef = (u >> 23) & 0xffu;
    const uint32_t frac = u & 0x7fffffu;
    if (ef == 0xffu) return (uint16_t)(s | (frac ? 0x7e00u : 0x7c00u));
    const int e16 = (int)ef - 112;
    uint32_t sig, sh;
    if (e16 > 0) {
        /* normal: keep 10 fraction bits, round on the 13 dropped ones */
        uint32_t h = ((uint32_t)e16 << 10) | (frac >> 13);
        const uint32_t rem = frac & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        if (h >= 0x7c00u) return (uint16_t)(s | 0x7c00u);
        return (uint16_t)(s | h);
    }
    if (e16 < -11 || ef == 0) return s;  /* below 2^-26: rounds to zero */
    sig = frac | 0x800000u;
    sh = (uint32_t)(14 - e16);          /* 14..25 */
    uint32_t h = sig >> sh;
    const uint32_t rem = sig & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(s | h);
}

/* double -> fp16 with one rounding (nearest-even): used where the oracle
 * carries more precision than the device and must not round twice. */
static uint16_t d2h_rne(double v) {
    if (isnan(v)) return 0x7e00u;
    const uint16_t s = signbit(v) ? 0x8000u : 0u;
    double a = fabs(v);
    if (a >= 65520.0) return (uint16_t)(s | 0x7c00u);
    int ex;
    (void)frexp(a, &ex);                 /* a = f * 2^ex, f in [0.5, 1) */
    int e = ex - 1;                      /* a in [2^e, 2^(e+1)) */
    if (e < -14) e = -14;                /* subnormal spacing 2^-24 */
    const double ulp = ldexp(1.0, e - 10);
    double q = a / ulp;                  /* exact: power-of-two scaling */
    double fl = floor(q);
    double r = q - fl;
    if (r > 0.5 || (r == 0.5 && fmod(fl, 2.0) != 0.0)) fl += 1.0;
    double res = fl * ulp;
    if (res >= 65520.0) return (uint16_t)(s | 0x7c00u);
    /* encode res (exactly representable) */
    if (res == 0.0) return s;
    int rx;
    (void)frexp(res, &rx);
    int re = rx - 1;
    if (re < -14) return (uint16_t)(s | (uint16_t)(res / ldexp(1.0, -24)));
    uint32_t mant = (uint32_t)(res / ldexp(1.0, re - 10)) - 1024u;
    return (uint16_t)(s | ((uint32_t)(re + 15) << 10) | mant);
}

void orc_f2h_array(const float* in, size_t n, uint16_t* out) {
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) out[i] = orc_f2h(in[i]);
}
void orc_f2h_rne_array(const float* in, size_t n, uint16_t* out) {
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) out[i] = orc_f2h_rne(in[i]);
}
void orc_h2f_array(const uint16_t* in, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_h2f(in[i]);
}

static inline float blk_half(const uint8_t* p) {
    return orc_h2f((uint16_t)(p[0] | (p[1] << 8)));
}

/* ------------------------------------------------------------------------ *
 * Q4_K: 144-byte super-block = d(f16) dmin(f16) scales[12] qs[128]
 * ------------------------------------------------------------------------ */

/* weight_loader.cpp:28-38 == kernels.cu:174-186: eight 6-bit (scale, min)
 * pairs packed in 12 bytes.  Pairs 0-3 sit in the low 6 bits of bytes 0-3
 * (scale) and 4-7 (min); pairs 4-7 take their low nibbles from bytes 8-11
 * and their top two bits from the spare high bits of bytes 0-7. */
void orc_q4k_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 0x3f;
        *m = q[j + 4] & 0x3f;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Element e of a Q4_K super-block, as the device computes it
 * (kernels.cu:213-230): group pair j = e/64, upper half of the pair when
 * e%64 >= 32; nibble from qs[32j + e%32]; value = d*sc*q - dmin*m in fp32.
 * d*sc*q and dmin*m are exact in fp32 (<= 21 and 17 significant bits), so
 * the one rounding is the subtraction and contraction cannot change it. */
static inline float q4k_value(const uint8_t* blk, int e) {
    const float d = blk_half(blk), dmin = blk_half(blk + 2);
    const int j = e >> 6, hi = (e & 63) >= 32;
    uint8_t sc, m;
    orc_q4k_scale_min(2 * j + hi, blk + 4, &sc, &m);
    const uint8_t b = blk[16 + 32 * j + (e & 31)];
    const int q = hi ? (b >> 4) : (b & 0x0f);
    const float dq = (d * (float)sc) * (float)q;
    const float mm = dmin * (float)m;
    return dq - mm;
}

/* weight_loader.cpp:147-237 (dequant_q4_k): same value, rounded with the
 * host rule (ties away).  The host computes (d*sc)*q - dmin*m with the same
 * exact products, so the fp32 value is q4k_value's. */
void orc_dequant_q4k_f16(const uint8_t* blocks, uint64_t count, uint16_t* out) {
    const uint64_t nb = (count + ORC_QK - 1) / ORC_QK;
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t* blk = blocks + b * ORC_Q4K_BYTES;
        for (int e = 0; e < ORC_QK; ++e) {
            const uint64_t idx = b * ORC_QK + (uint64_t)e;
            if (idx < count) out[idx] = orc_f2h(q4k_value(blk, e));
        }
    }
}

void orc_dequant_q4k_f32(const uint8_t* blocks, uint64_t count, float* out) {
    const uint64_t nb = (count + ORC_QK - 1) / ORC_QK;
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t* blk = blocks + b * ORC_Q4K_BYTES;
        for (int e = 0; e < ORC_QK; ++e) {
            const uint64_t idx = b * ORC_QK + (uint64_t)e;
            if (idx < count) out[idx] = q4k_value(blk, e);
        }
    }
}

/* ------------------------------------------------------------------------ *
 * Q6_K: 210-byte super-block = ql[128] qh[64] scales int8[16] d(f16)
 * ------------------------------------------------------------------------ */

/* kernels.cu:134-172 (dequant_q6k_value) and weight_loader.cpp:265-319:
 * element e: half h = e/128, part = (e%128)/32, i = e%32.  Low 4 bits from
 * ql[64h + 32*(part&1) + i] (low nibble for part < 2, high nibble else),
 * high 2 bits from qh[32h + i] >> 2*part; q = q6 - 32; scale index
 * 8h + i/16 + 2*part.  (d*sc)*q is exact in fp32 (<= 23 significant bits). */
static inline float q6k_value(const uint8_t* blk, int e) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const float d = blk_half(blk + 208);
    const int h = e >> 7, part = (e & 127) >> 5, i = e & 31;
    const uint8_t lb = ql[64 * h + 32 * (part & 1) + i];
    const int lo = part < 2 ? (lb & 0x0f) : (lb >> 4);
    const int hi2 = (qh[32 * h + i] >> (2 * part)) & 3;
    const int q = (lo | (hi2 << 4)) - 32;
    return (d * (float)sc[8 * h + i / 16 + 2 * part]) * (float)q;
}

/* weight_loader.cpp:240-323 (dequant_q6_k): host rule rounding. */
void orc_dequant_q6k_f16(const uint8_t* blocks, uint64_t count, uint16_t* out) {
    const uint64_t nb = (count + ORC_QK - 1) / ORC_QK;
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t* blk = blocks + b * ORC_Q6K_BYTES;
        for (int e = 0; e < ORC_QK; ++e) {
            const uint64_t idx = b * ORC_QK + (uint64_t)e;
            if (idx < count) out[idx] = orc_f2h(q6k_value(blk, e));
        }
    }
}

void orc_dequant_q6k_f32(const uint8_t* blocks, uint64_t count, float* out) {
    const uint64_t nb = (count + ORC_QK - 1) / ORC_QK;
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t* blk = blocks + b * ORC_Q6K_BYTES;
        for (int e = 0; e < ORC_QK; ++e) {
            const uint64_t idx = b * ORC_QK + (uint64_t)e;
            if (idx < count) out[idx] = q6k_value(blk, e);
        }
    }
}

/* ------------------------------------------------------------------------ *
 * GEMV
 * ------------------------------------------------------------------------ */

/* All 256 values of one block, q4k_value(blk, e) for e = 0..255, with the
 * block's d, dmin and (scale, min) pairs read once per block instead of once
 * per value.  Same fp32 expressions, so the same values. */
static void q4k_block_values(const uint8_t* blk, float* out) {
    const float d = blk_half(blk), dmin = blk_half(blk + 2);
    for (int j = 0; j < 4; ++j) {
        uint8_t sc0, m0, sc1, m1;
        orc_q4k_scale_min(2 * j, blk + 4, &sc0, &m0);
        orc_q4k_scale_min(2 * j + 1, blk + 4, &sc1, &m1);
        const float ds0 = d * (float)sc0, mm0 = dmin * (float)m0;
        const float ds1 = d * (float)sc1, mm1 = dmin * (float)m1;
        const uint8_t* qs = blk + 16 + 32 * j;
        for (int i = 0; i < 32; ++i) {
            out[64 * j + i] = ds0 * (float)(qs[i] & 0x0f) - mm0;
            out[64 * j + 32 + i] = ds1 * (float)(qs[i] >> 4) - mm1;
        }
    }
}

/* q6k_value(blk, e) for e = 0..255 (e = 128h + 32part + i). */
static void q6k_block_values(const uint8_t* blk, float* out) {
    const float d = blk_half(blk + 208);
    const int8_t* sc = (const int8_t*)(blk + 192);
    for (int h = 0; h < 2; ++h)
        for (int part = 0; part < 4; ++part)
            for (int i = 0; i < 32; ++i) {
                const uint8_t lb = blk[64 * h + 32 * (part & 1) + i];
                const int lo = part < 2 ? (lb & 0x0f) : (lb >> 4);
                const int hi2 = (blk[128 + 32 * h + i] >> (2 * part)) & 3;
                const int q = (lo | (hi2 << 4)) - 32;
                out[128 * h + 32 * part + i] = (d * (float)sc[8 * h + i / 16 + 2 * part]) * (float)q;
            }
}

/* kernels.cu:195-251 / 253-291 / 293-338: y[row] = sum over the row's
 * super-blocks of value(e) * x[256*b + e], weights kept in fp32 (never
 * rounded to fp16).  Accumulated here in double, one running sum per row in
 * element order: acc += w*x with the product exact in double (24 + 11
 * significant bits) and the add the only rounding, so the result depends
 * on nothing but that order.  Four rows are decoded and summed side by side
 * (each with its own sum) so the adds of different rows overlap. */
#define ORC_ROW_GROUP 4
static void matvec_kquant(int q6, const uint8_t* w, const uint16_t* x, double* y, int in_f, int out_f, int nthreads) {
    const int nb = in_f / ORC_QK;
    const size_t bb = q6 ? ORC_Q6K_BYTES : ORC_Q4K_BYTES;
    double* xd = (double*)malloc((size_t)(in_f > 0 ? in_f : 1) * sizeof(double));
    for (int k = 0; k < in_f; ++k) xd[k] = (double)orc_h2f(x[k]);
    const int groups = (out_f + ORC_ROW_GROUP - 1) / ORC_ROW_GROUP;
    #pragma omp parallel for schedule(static) num_threads(pick_threads(nthreads))
    for (int g = 0; g < groups; ++g) {
        const int r0 = g * ORC_ROW_GROUP;
        const int nr = out_f - r0 < ORC_ROW_GROUP ? out_f - r0 : ORC_ROW_GROUP;
        float v[ORC_ROW_GROUP][ORC_QK];
        double acc[ORC_ROW_GROUP] = {0.0, 0.0, 0.0, 0.0};
        for (int b = 0; b < nb; ++b) {
            for (int r = 0; r < nr; ++r) {
                const uint8_t* blk = w + ((size_t)(r0 + r) * nb + b) * bb;
                if (q6) q6k_block_values(blk, v[r]);
                else q4k_block_values(blk, v[r]);
            }
            const double* xb = xd + (size_t)b * ORC_QK;
            if (nr == ORC_ROW_GROUP) {
                double a0 = acc[0], a1 = acc[1], a2 = acc[2], a3 = acc[3];
                for (int e = 0; e < ORC_QK; ++e) {
                    a0 += (double)v[0][e] * xb[e];
                    a1 += (double)v[1][e] * xb[e];
                    a2 += (double)v[2][e] * xb[e];
                    a3 += (double)v[3][e] * xb[e];
                }
                acc[0] = a0; acc[1] = a1; acc[2] = a2; acc[3] = a3;
            } else {
                for (int r = 0; r < nr; ++r)
                    for (int e = 0; e < ORC_QK; ++e) acc[r] += (double)v[r][e] * xb[e];
            }
        }
        for (int r = 0; r < nr; ++r) y[r0 + r] = acc[r];
    }
    free(xd);
}

void orc_matvec_q4k(const uint8_t* w, const uint16_t* x, double* y, int in_f, int out_f, int nthreads) {
    matvec_kquant(0, w, x, y, in_f, out_f, nthreads);
}

void orc_matvec_q6k(const uint8_t* w, const uint16_t* x, double* y, int in_f, int out_f, int nthreads) {
    matvec_kquant(1, w, x, y, in_f, out_f, nthreads);
}

/* CPU baseline (i): the reference's host arithmetic -- repo dequant of the
 * row to fp16 bits (host rule), then an fp32 dot -- once per call. */
void orc_matvec_q4k_f16dot(const uint8_t* w, const uint16_t* x, float* y, int in_f, int out_f, int nthreads) {
    const int nb = in_f / ORC_QK;
    #pragma omp parallel num_threads(pick_threads(nthreads))
    {
        uint16_t* tmp = (uint16_t*)malloc((size_t)in_f * 2);
        float* xf = (float*)malloc((size_t)in_f * 4);
        for (int k = 0; k < in_f; ++k) xf[k] = orc_h2f(x[k]);
        #pragma omp for schedule(static)
        for (int r = 0; r < out_f; ++r) {
            orc_dequant_q4k_f16(w + (size_t)r * nb * ORC_Q4K_BYTES, (uint64_t)in_f, tmp);
            float acc = 0.0f;
            for (int k = 0; k < in_f; ++k) acc += orc_h2f(tmp[k]) * xf[k];
            y[r] = acc;
        }
        free(tmp);
        free(xf);
    }
}

void orc_matvec_q6k_f16dot(const uint8_t* w, const uint16_t* x, float* y, int in_f, int out_f, int nthreads) {
    const int nb = in_f / ORC_QK;
    #pragma omp parallel num_threads(pick_threads(nthreads))
    {
        uint16_t* tmp = (uint16_t*)malloc((size_t)in_f * 2);
        float* xf = (float*)malloc((size_t)in_f * 4);
        for (int k = 0; k < in_f; ++k) xf[k] = orc_h2f(x[k]);
        #pragma omp for schedule(static)
        for (int r = 0; r < out_f; ++r) {
            orc_dequant_q6k_f16(w + (size_t)r * nb * ORC_Q6K_BYTES, (uint64_t)in_f, tmp);
            float acc = 0.0f;
            for (int k = 0; k < in_f; ++k) acc += orc_h2f(tmp[k]) * xf[k];
            y[r] = acc;
        }
        free(tmp);
        free(xf);
    }
}

/* CPU baseline (ii): dot over weights already dequantised to fp16 bits
 * (kernels.cu:381-471 semantics, fp32 accumulation). */
void orc_matvec_f16(const uint16_t* w, const uint16_t* x, float* y, int in_f, int out_f, int nthreads) {
    #pragma omp parallel num_threads(pick_threads(nthreads))
    {
        float* xf = (float*)malloc((size_t)in_f * 4);
        for (int k = 0; k < in_f; ++k) xf[k] = orc_h2f(x[k]);
        #pragma omp for schedule(static)
        for (int r = 0; r < out_f; ++r) {
            const uint16_t* row = w + (size_t)r * in_f;
            float acc = 0.0f;
            for (int k = 0; k < in_f; ++k) acc += orc_h2f(row[k]) * xf[k];
            y[r] = acc;
        }
        free(xf);
    }
}

/* ------------------------------------------------------------------------ *
 * embedding
 * ------------------------------------------------------------------------ */

/* kernels.cu:340-378 gathers row token_id of a Q6_K table, dequantises each
 * value in fp32 (dequant_q6k_value) and stores it with __float2half, i.e.
 * rounded nearest-even (kernels.cu:21-24). */
void orc_embed_q6k(const uint8_t* table, int32_t token_id, uint16_t* out, int hidden) {
    const int nb = hidden / ORC_QK;
    float* v = (float*)malloc((size_t)hidden * sizeof(float));
    orc_dequant_q6k_f32(table + (size_t)token_id * nb * ORC_Q6K_BYTES, (uint64_t)hidden, v);
    orc_f2h_rne_array(v, (size_t)hidden, out);
    free(v);
}

/* ------------------------------------------------------------------------ *
 * decode attention
 * ------------------------------------------------------------------------ */

/* kernels.cu:545-649: for query head h (kv head h / (heads/kv_heads)) and
 * positions t = 0..position: s_t = (q_h . K[t]) / sqrt(hd); softmax over t
 * (max-subtracted); out = sum_t p_t V[t].  Caches are [pos][kv_heads][hd]
 * (kernels.cu:524-533).  Double precision throughout. */
void orc_attention(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                   int position, int heads, int kv_heads, int hd, double* out) {
    const int group = heads / kv_heads;
    const int L = position + 1;
    const double scale = 1.0 / sqrt((double)hd);
    /* heads are independent and each is summed serially, so the result does
     * not depend on the thread count */
    #pragma omp parallel for schedule(dynamic, 1) if ((long long)L * heads >= 65536)
    for (int h = 0; h < heads; ++h) {
        double* s = (double*)malloc((size_t)L * sizeof(double));
        const int kvh = h / group;
        double mx = -INFINITY;
        for (int t = 0; t < L; ++t) {
            const uint16_t* k = kc + ((size_t)t * kv_heads + kvh) * hd;
            double acc = 0.0;
            for (int d = 0; d < hd; ++d) acc += (double)orc_h2f(q[h * hd + d]) * (double)orc_h2f(k[d]);
            s[t] = acc * scale;
            if (s[t] > mx) mx = s[t];
        }
        double den = 0.0;
        for (int t = 0; t < L; ++t) { s[t] = exp(s[t] - mx); den += s[t]; }
        /* positions outer, dims inner: each dim's sum runs over t in order */
        double* acc = (double*)calloc((size_t)hd, sizeof(double));
        for (int t = 0; t < L; ++t) {
            const uint16_t* v = vc + ((size_t)t * kv_heads + kvh) * hd;
            for (int d = 0; d < hd; ++d) acc[d] += s[t] * (double)orc_h2f(v[d]);
        }
        for (int d = 0; d < hd; ++d) out[h * hd + d] = acc[d] / den;
        free(acc);
        free(s);
    }
}

/* Float version for the CPU baseline: same algorithm, fp32 scores and
 * softmax like the reference kernels, parallel over query heads. */
void orc_attention_f32(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                       int position, int heads, int kv_heads, int hd, float* out, int nthreads) {
    const int group = heads / kv_heads;
    const int L = position + 1;
    const float scale = 1.0f / sqrtf((float)hd);
    #pragma omp parallel num_threads(pick_threads(nthreads))
    {
        float* s = (float*)malloc((size_t)L * sizeof(float));
        float* qf = (float*)malloc((size_t)hd * sizeof(float));
        float* acc = (float*)malloc((size_t)hd * sizeof(float));
        #pragma omp for schedule(static)
        for (int h = 0; h < heads; ++h) {
            const int kvh = h / group;
            for (int d = 0; d < hd; ++d) qf[d] = orc_h2f(q[h * hd + d]);
            float mx = -INFINITY;
            for (int t = 0; t < L; ++t) {
                const uint16_t* k = kc + ((size_t)t * kv_heads + kvh) * hd;
                float a = 0.0f;
                for (int d = 0; d < hd; ++d) a += qf[d] * orc_h2f(k[d]);
                s[t] = a * scale;
                if (s[t] > mx) mx = s[t];
            }
            float den = 0.0f;
            for (int d = 0; d < hd; ++d) acc[d] = 0.0f;
            for (int t = 0; t < L; ++t) {
                const float p = expf(s[t] - mx);
                den += p;
                const uint16_t* v = vc + ((size_t)t * kv_heads + kvh) * hd;
                for (int d = 0; d < hd; ++d) acc[d] += p * orc_h2f(v[d]);
            }
            for (int d = 0; d < hd; ++d) out[h * hd + d] = acc[d] / den;
        }
        free(s);
        free(qf);
        free(acc);
    }
}

/* ------------------------------------------------------------------------ *
 * remaining forward_token ops
 * ------------------------------------------------------------------------ */

/* kernels.cu:73-92: out = fp16(x * rsqrt(mean(x^2) + eps) * w). */
void orc_rms_norm(const uint16_t* in, const uint16_t* w, uint16_t* out, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) { const double v = orc_h2f(in[i]); ss += v * v; }
    const double inv = 1.0 / sqrt(ss / (double)n + (double)eps);
    for (int i = 0; i < n; ++i) out[i] = d2h_rne((double)orc_h2f(in[i]) * inv * (double)orc_h2f(w[i]));
}

/* kernels.cu:95-124: the same per head, weight shared by all heads. */
void orc_rms_norm_heads(const uint16_t* in, const uint16_t* w, uint16_t* out, int heads, int hd, float eps) {
    for (int h = 0; h < heads; ++h) orc_rms_norm(in + (size_t)h * hd, w, out + (size_t)h * hd, hd, eps);
}

/* kernels.cu:485-521: NeoX rotation of the pair (i, i + hd/2) by
 * angle = position * theta^(-2i/hd).  The angle is formed in fp32 from an
 * fp32 inverse frequency, as the reference does; sin/cos of that angle are
 * taken in double. */
void orc_rope(uint16_t* data, int heads, int hd, int position, float theta) {
    const int half = hd / 2;
    for (int h = 0; h < heads; ++h) {
        for (int i = 0; i < half; ++i) {
            const float inv_freq = (float)pow((double)theta, -(double)(2 * i) / (double)hd);
            const float angle = (float)position * inv_freq;
            const double s = sin((double)angle), c = cos((double)angle);
            const double x0 = orc_h2f(data[h * hd + i]);
            const double x1 = orc_h2f(data[h * hd + half + i]);
            data[h * hd + i] = d2h_rne(x0 * c - x1 * s);
            data[h * hd + half + i] = d2h_rne(x0 * s + x1 * c);
        }
    }
}

/* kernels.cu:474-482: out = fp16(silu(g) * u). */
void orc_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int n) {
    for (int i = 0; i < n; ++i) {
        const double g = orc_h2f(gate[i]);
        out[i] = d2h_rne(g / (1.0 + exp(-g)) * (double)orc_h2f(up[i]));
    }
}

/* kernels.cu:53-59: target = fp16(target + delta), sum formed in fp32. */
void orc_add_inplace(uint16_t* t, const uint16_t* d, int n) {
    for (int i = 0; i < n; ++i) t[i] = orc_f2h_rne(orc_h2f(t[i]) + orc_h2f(d[i]));
}

/* kernels.cu:524-533: cache[position * kv_size + i] = v[i]. */
void orc_store_kv(const uint16_t* k, const uint16_t* v, uint16_t* kc, uint16_t* vc, int position, int kv_size) {
    memcpy(kc + (size_t)position * kv_size, k, (size_t)kv_size * 2);
    memcpy(vc + (size_t)position * kv_size, v, (size_t)kv_size * 2);
}

/* qwen_model.cpp:455-463: first strictly greater finite value wins; all
 * non-finite -> 0. */
int32_t orc_argmax(const float* logits, int n) {
    float best = -INFINITY;
    int32_t id = 0;
    for (int i = 0; i < n; ++i) {
        const float v = logits[i];
        if (isfinite(v) && v > best) { best = v; id = i; }
    }
    return id;
}

/* ------------------------------------------------------------------------ *
 * one decode step (qwen_model.cpp:239-419)
 * ------------------------------------------------------------------------ */

/* y = W x in double for any supported weight type (fp16 weights: the
 * DequantizeToFp16 path's matvec_fp16, kernels.cu:381-471). */
static void matvec_any(const OrcMatrix* w, const uint16_t* x, double* y, int in_f, int out_f) {
    if (w->type == ORC_Q4K) {
        orc_matvec_q4k((const uint8_t*)w->data, x, y, in_f, out_f, 0);
    } else if (w->type == ORC_Q6K) {
        orc_matvec_q6k((const uint8_t*)w->data, x, y, in_f, out_f, 0);
    } else {
        const uint16_t* wf = (const uint16_t*)w->data;
#pragma omp parallel for schedule(static)
        for (int r = 0; r < out_f; ++r) {
            double acc = 0.0;
            for (int k = 0; k < in_f; ++k)
                acc += (double)orc_h2f(wf[(size_t)r * in_f + k]) * (double)orc_h2f(x[k]);
            y[r] = acc;
        }
    }
}

/* linear_backend.cpp:19-61 then add_bias_if_present (qwen_model.cpp:28-33):
 * fp16 output, then an fp32 bias add stored as fp16. */
static void linear(const OrcMatrix* w, const uint16_t* bias, const uint16_t* x, int in_f, int out_f, uint16_t* y,
                   double* tmp) {
    matvec_any(w, x, tmp, in_f, out_f);
    for (int i = 0; i < out_f; ++i) y[i] = d2h_rne(tmp[i]);
    if (bias) orc_add_inplace(y, bias, out_f);
}

/* The embedding and every layer of one step (qwen_model.cpp:256-374): the
 * caches gain this position and x (hidden fp16) holds the residual stream
 * that the final norm reads. */
static void forward_layers(const OrcModel* m, uint16_t* const* caches, int32_t token, int position, uint16_t* x) {
    const int H = m->hidden, hd = m->head_dim, nq = m->heads * hd, nkv = m->kv_heads * hd, ff = m->ff;
    const size_t big = (size_t)ff + (size_t)nq + H;
    uint16_t* norm = (uint16_t*)malloc((size_t)H * 2);
    uint16_t* q = (uint16_t*)malloc((size_t)nq * 2);
    uint16_t* k = (uint16_t*)malloc((size_t)nkv * 2);
    uint16_t* v = (uint16_t*)malloc((size_t)nkv * 2);
    uint16_t* att = (uint16_t*)malloc((size_t)nq * 2);
    uint16_t* proj = (uint16_t*)malloc((size_t)H * 2);
    uint16_t* gate = (uint16_t*)malloc((size_t)ff * 2);
    uint16_t* up = (uint16_t*)malloc((size_t)ff * 2);
    uint16_t* act = (uint16_t*)malloc((size_t)ff * 2);
    double* tmp = (double*)malloc(big * sizeof(double));

    /* token embedding (qwen_model.cpp:256-268) */
    if (m->token_embd.type == ORC_Q6K)
        orc_embed_q6k((const uint8_t*)m->token_embd.data, token, x, H);
    else
        memcpy(x, (const uint16_t*)m->token_embd.data + (size_t)token * H, (size_t)H * 2);

    for (int l = 0; l < m->n_layers; ++l) {
        const OrcLayer* L = &m->layers[l];
        uint16_t* kc = caches[2 * l];
        uint16_t* vc = caches[2 * l + 1];
        orc_rms_norm(x, L->attn_norm, norm, H, m->eps);
        linear(&L->q, L->q_bias, norm, H, nq, q, tmp);
        linear(&L->k, L->k_bias, norm, H, nkv, k, tmp);
        linear(&L->v, L->v_bias, norm, H, nkv, v, tmp);
        if (L->q_norm) orc_rms_norm_heads(q, L->q_norm, q, m->heads, hd, m->eps);
        if (L->k_norm) orc_rms_norm_heads(k, L->k_norm, k, m->kv_heads, hd, m->eps);
        orc_rope(q, m->heads, hd, position, m->theta);
        orc_rope(k, m->kv_heads, hd, position, m->theta);
        orc_store_kv(k, v, kc, vc, position, nkv);
        orc_attention(q, kc, vc, position, m->heads, m->kv_heads, hd, tmp);
        for (int i = 0; i < nq; ++i) att[i] = d2h_rne(tmp[i]);
        linear(&L->o, L->o_bias, att, nq, H, proj, tmp);
        orc_add_inplace(x, proj, H);
        orc_rms_norm(x, L->ffn_norm, norm, H, m->eps);
        linear(&L->gate, L->gate_bias, norm, H, ff, gate, tmp);
        linear(&L->up, L->up_bias, norm, H, ff, up, tmp);
        orc_swiglu(gate, up, act, ff);
        linear(&L->down, L->down_bias, act, ff, H, proj, tmp);
        orc_add_inplace(x, proj, H);
    }
    free(norm); free(q); free(k); free(v); free(att); free(proj);
    free(gate); free(up); free(act); free(tmp);
}

int32_t orc_forward_token(const OrcModel* m, uint16_t* const* caches, int32_t token, int position, float* logits) {
    const int H = m->hidden;
    uint16_t* x = (uint16_t*)malloc((size_t)H * 2);
    uint16_t* norm = (uint16_t*)malloc((size_t)H * 2);
    double* tmp = (double*)malloc((size_t)m->vocab * sizeof(double));
    forward_layers(m, caches, token, position, x);
    /* final norm, fp32 logits, greedy pick (qwen_model.cpp:385-419, 448-465) */
    orc_rms_norm(x, m->output_norm, norm, H, m->eps);
    matvec_any(&m->output, norm, tmp, H, m->vocab);
    float* lg = logits ? logits : (float*)malloc((size_t)m->vocab * sizeof(float));
    for (int i = 0; i < m->vocab; ++i) lg[i] = (float)tmp[i];
    const int32_t next = orc_argmax(lg, m->vocab);
    if (!logits) free(lg);
    free(x); free(norm); free(tmp);
    return next;
}

void orc_prefill_token(const OrcModel* m, uint16_t* const* caches, int32_t token, int position) {
    uint16_t* x = (uint16_t*)malloc((size_t)m->hidden * 2);
    forward_layers(m, caches, token, position, x);
    free(x);
}
