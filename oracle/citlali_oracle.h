/*
 * citlali_oracle.h -- CPU restatement of the Citlali decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the parity tests,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py compare the
 * HIP path against.  Nothing in the product (libcitlali_hip.so,
 * libcitlali.so, pycitlali) links, loads or calls it.
 *
 * Every function names the reference file:line whose behaviour it restates
 * (paths relative to the reference repository root).  Pinning of each
 * function (what independent evidence checks the restatement):
 *   orc_f2h / orc_h2f        -- closed-form spec over all 2^32 / 2^16 inputs,
 *                               known answers, the compiled reference
 *                               (oracle/_ref) and the committed golden vectors.
 *   orc_f2h_rne              -- IEEE binary16 round-to-nearest-even; checked
 *                               against numpy's float32->float16 cast.
 *   orc_dequant_q4k/q6k_f16  -- golden vectors written by the compiled
 *                               reference (tests/golden), closed forms.
 *   orc_dequant_*_f32        -- one-hot / closed-form checks and consistency
 *                               with the f16 routines (f16(f32 value) must
 *                               equal the f16 routine bit for bit).
 *   orc_matvec_*             -- linearity, row sums with x = 1, one-hot x,
 *                               brute-force numpy dot on small shapes.
 *   orc_attention            -- L = 1 (out = V[0]), q = 0 (mean of V),
 *                               GQA head equality, numpy softmax on small
 *                               shapes.
 *   orc_embed_q6k            -- numpy's nearest-even cast of the f32 row.
 *   orc_rms_norm(_heads), orc_rope, orc_swiglu, orc_add_inplace,
 *   orc_store_kv, orc_argmax -- known answers, closed forms (unit vectors,
 *                               one-hot rotations, silu(0)), numpy fp32
 *                               adds, tie / NaN rules (test_oracle_forward).
 *   orc_forward_token        -- composition of the pinned pieces; zeroed
 *                               residual branches, an inert second layer
 *                               and cache dependence (tests/cpp, cpu mode).
 */
#ifndef CITLALI_ORACLE_H
#define CITLALI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK 256
#define ORC_Q4K_BYTES 144
#define ORC_Q6K_BYTES 210

/* ---- fp16 conversion (dtype.cpp:76-176) ---------------------------------- */
uint16_t orc_f2h(float v);          /* reference host rule: nearest, ties away, NaN -> Inf */
float    orc_h2f(uint16_t h);       /* exact widening */
uint16_t orc_f2h_rne(float v);      /* IEEE nearest-even (device __float2half rule) */
void     orc_f2h_array(const float* in, size_t n, uint16_t* out);
void     orc_f2h_rne_array(const float* in, size_t n, uint16_t* out);
void     orc_h2f_array(const uint16_t* in, size_t n, float* out);

/* ---- Q4_K / Q6_K dequantisation ------------------------------------------ */
void orc_q4k_scale_min(int j, const uint8_t* scales, uint8_t* sc, uint8_t* m);
/* host load-time dequant to fp16 bits (weight_loader.cpp:147-237, 240-323) */
void orc_dequant_q4k_f16(const uint8_t* blocks, uint64_t count, uint16_t* out);
void orc_dequant_q6k_f16(const uint8_t* blocks, uint64_t count, uint16_t* out);
/* device in-kernel value before any rounding (kernels.cu:134-172, 195-233) */
void orc_dequant_q4k_f32(const uint8_t* blocks, uint64_t count, float* out);
void orc_dequant_q6k_f32(const uint8_t* blocks, uint64_t count, float* out);

/* ---- GEMV (kernels.cu:195-338) ------------------------------------------- *
 * y[r] = sum_k W_f32[r,k] * x[k] accumulated in double, returned as double.
 * W row-major [out][in/256] super-blocks.  nthreads <= 0 -> all cores.     */
void orc_matvec_q4k(const uint8_t* w, const uint16_t* x, double* y, int in_features, int out_features, int nthreads);
void orc_matvec_q6k(const uint8_t* w, const uint16_t* x, double* y, int in_features, int out_features, int nthreads);
/* CPU-baseline flavours, float accumulation like the reference's "repo dequant
 * to fp16, then fp32 dot": (i) dequant per call, (ii) pre-dequantised fp16.  */
void orc_matvec_q4k_f16dot(const uint8_t* w, const uint16_t* x, float* y, int in_features, int out_features, int nthreads);
void orc_matvec_q6k_f16dot(const uint8_t* w, const uint16_t* x, float* y, int in_features, int out_features, int nthreads);
void orc_matvec_f16(const uint16_t* w, const uint16_t* x, float* y, int in_features, int out_features, int nthreads);

/* ---- embedding (kernels.cu:340-378): the fp32 value, rounded nearest-even - */
void orc_embed_q6k(const uint8_t* table, int32_t token_id, uint16_t* out, int hidden);

/* ---- decode attention (kernels.cu:545-649) ------------------------------- *
 * q [heads][hd] fp16; caches [max_ctx][kv_heads][hd] fp16; positions
 * 0..position inclusive; scale 1/sqrt(hd); fp32-or-better softmax.
 * out [heads][hd] as double (unrounded).                                    */
void orc_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                   int position, int heads, int kv_heads, int head_dim, double* out);
/* float-accumulating multi-threaded version used as the CPU baseline */
void orc_attention_f32(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                       int position, int heads, int kv_heads, int head_dim, float* out, int nthreads);

/* ---- the rest of forward_token (kernels.cu:53-124, 474-533) -------------- */
void orc_rms_norm(const uint16_t* in, const uint16_t* w, uint16_t* out, int n, float eps);
void orc_rms_norm_heads(const uint16_t* in, const uint16_t* w, uint16_t* out, int heads, int head_dim, float eps);
void orc_rope(uint16_t* data, int heads, int head_dim, int position, float theta);
void orc_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int n);
void orc_add_inplace(uint16_t* target, const uint16_t* delta, int n);
void orc_store_kv(const uint16_t* k, const uint16_t* v, uint16_t* kc, uint16_t* vc, int position, int kv_size);
/* greedy argmax with the host tie rule (qwen_model.cpp:455-463) */
int32_t orc_argmax(const float* logits, int n);

/* ---- one decode step of the model (qwen_model.cpp:239-419) -------------- *
 * Composes the routines above in the reference's order with its fp16 store
 * points: every GEMV / norm / rope / attention / swiglu / add result is
 * stored as fp16 (nearest-even) before the next operation reads it; the
 * logits stay fp32.  No remote layers.                                     */
#define ORC_F16 1
#define ORC_Q4K 12
#define ORC_Q6K 14
typedef struct {
    int type;            /* ORC_F16, ORC_Q4K or ORC_Q6K */
    const void* data;    /* [rows = out][in] */
} OrcMatrix;
typedef struct {
    const uint16_t* attn_norm;
    OrcMatrix q, k, v, o;
    const uint16_t *q_bias, *k_bias, *v_bias, *o_bias;   /* NULL when absent */
    const uint16_t *q_norm, *k_norm;                      /* NULL when absent */
    const uint16_t* ffn_norm;
    OrcMatrix gate, up, down;
    const uint16_t *gate_bias, *up_bias, *down_bias;      /* NULL when absent */
} OrcLayer;
typedef struct {
    int hidden, heads, kv_heads, head_dim, ff, n_layers, vocab, max_ctx;
    float eps, theta;
    OrcMatrix token_embd;   /* ORC_Q6K or ORC_F16, [vocab][hidden] */
    const uint16_t* output_norm;
    OrcMatrix output;       /* ORC_Q6K or ORC_F16, [vocab][hidden] */
    const OrcLayer* layers;
} OrcModel;
/* caches: 2 * n_layers caller-owned fp16 arrays [max_ctx][kv_heads*head_dim]
 * (k0, v0, k1, v1, ...).  logits (vocab floats) may be NULL.  Returns the
 * greedy token of the fp32 logits (orc_argmax rule). */
int32_t orc_forward_token(const OrcModel* m, uint16_t* const* caches, int32_t token, int position, float* logits);
/* The same step without the final norm and output GEMV: for prompt positions
 * whose logits nobody reads (the caches are filled identically). */
void orc_prefill_token(const OrcModel* m, uint16_t* const* caches, int32_t token, int position);

/* ---- misc ---------------------------------------------------------------- */
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
