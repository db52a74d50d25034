/*
 * citlali_hip.h -- C ABI of the MI355X (gfx950) decode hot path.
 *
 * This is the drop-in boundary that replaces the reference's CUDA layer
 * (include/citlali/compute/cuda/{kernels.h,tensor.h,cuda_utils.h} and
 * src/compute/cuda/{kernels.cu,tensor.cu}).  Plain pointers and sizes only.
 *
 * Conventions (same as the reference's launch_* functions, kernels.h:8-61):
 *  - fp16 values are uint16_t bit patterns, quantised weights raw GGUF
 *    super-blocks (uint8_t), fp32 values float; all pointers are device
 *    pointers unless a parameter says "host".
 *  - weights are row-major [out_features][in_features/256] super-blocks.
 *  - every call returns CITLALI_OK or an error code; the message of the last
 *    error of the calling thread is citlali_hip_last_error().  Argument
 *    checks run before anything touches the GPU.  HIP failures read
 *    "HIP error at <file>:<line> for <expr>: <message>" (the shape of the
 *    reference's CITLALI_CUDA_CHECK, cuda_utils.h:17-22).
 *  - launches are asynchronous on the library's current stream (default: the
 *    null stream, like the reference's <<<>>> launches); D2H copies and
 *    citlali_hip_synchronize() wait for it.
 *  - alignment: quantised Q4_K weights and x vectors 16-byte aligned, Q6_K
 *    weights 4-byte aligned (any hipMalloc'd buffer qualifies).
 */
#ifndef CITLALI_HIP_H
#define CITLALI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CITLALI_OK 0
#define CITLALI_ERR_INVALID 1     /* rejected argument, nothing launched */
#define CITLALI_ERR_UNSUPPORTED 2 /* valid for the reference, not built here */
#define CITLALI_ERR_HIP 3         /* HIP runtime error */

#define CITLALI_HIP_ABI_VERSION 1

/* ---- errors and runtime ------------------------------------------------- */

/* Replaces check_cuda/CITLALI_CUDA_CHECK (cuda_utils.h:17-26): message of the
 * calling thread's last failed call ("" if none). */
const char* citlali_hip_last_error(void);
int citlali_hip_abi_version(void);

/* Selects the device for this thread (the reference always uses device 0). */
int citlali_hip_init(int device);
int citlali_hip_device_count(int* count);

/* Stream used by every launch (hipStream_t; NULL = null stream, the
 * reference's legacy default stream). */
int citlali_hip_set_stream(void* stream);
void* citlali_hip_get_stream(void);

/* Replaces QwenModel::synchronize's cudaDeviceSynchronize
 * (qwen_model.cpp:443-445): waits for the current stream and reports any
 * asynchronous kernel fault. */
int citlali_hip_synchronize(void);

/* ---- device memory: DeviceBuffer (tensor.h:10-54, tensor.cu:49-104) ------ */

int citlali_hip_malloc(void** ptr, size_t bytes);              /* tensor.cu:49-59 (bytes == 0 -> *ptr = NULL) */
int citlali_hip_free(void* ptr);                               /* tensor.cu:67-73 */
/* tensor.cu:76-78; returns once the bytes are on the device.  Copies of 8 MB
 * and more go through two pinned 8 MB staging buffers per device (allocated
 * on first use, kept until the process ends), host threads filling one while
 * the DMA engine drains the other. */
int citlali_hip_memcpy_h2d(void* dst, const void* host_src, size_t bytes);
int citlali_hip_memcpy_d2h(void* host_dst, const void* src, size_t bytes); /* tensor.cu:88-90, waits */
int citlali_hip_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* cuda_zero (kernels.h:8, kernels.cu:655-657); a fill kernel, so it is safe
 * inside captured graphs. */
int citlali_hip_zero(void* ptr, size_t bytes);

/* ---- hot path: fused dequant GEMV ---------------------------------------- *
 * y[r] = sum_k W[r,k] x[k], W dequantised in fp32 (never rounded to fp16),
 * fp32 accumulation.  in_features must be a positive multiple of 256 (the
 * reference truncates silently, kernels.cu:204; this ABI rejects it) and at
 * most CITLALI_MAX_IN_FEATURES. */
#define CITLALI_MAX_IN_FEATURES 28672

/* launch_matvec_q4k (kernels.h:26, kernels.cu:772-776); y fp16 (RNE) */
int citlali_hip_matvec_q4k(const uint8_t* w, const uint16_t* x, uint16_t* y, int in_features, int out_features);
/* Q4_K with fp32 output: no reference launcher; same kernel, fp32 store
 * (the fp32-output form the reference has for Q6_K, kernels.h:30). */
int citlali_hip_matvec_q4k_to_float(const uint8_t* w, const uint16_t* x, float* y, int in_features,
                                    int out_features);
/* launch_matvec_q6k (kernels.h:28, kernels.cu:779-783); y fp16 (RNE) */
int citlali_hip_matvec_q6k(const uint8_t* w, const uint16_t* x, uint16_t* y, int in_features, int out_features);
/* launch_matvec_q6k_to_float (kernels.h:30, kernels.cu:786-796); logits */
int citlali_hip_matvec_q6k_to_float(const uint8_t* w, const uint16_t* x, float* y, int in_features,
                                    int out_features);

/* launch_embed_q6k (kernels.h:32, kernels.cu:340-378, 670-683): row
 * token_id of a Q6_K table -> fp16, the exact fp32 value rounded
 * nearest-even as the reference kernel's __float2half store does. */
int citlali_hip_embed_q6k(const uint8_t* table, int32_t token_id, uint16_t* out, int hidden);

/* ---- hot path: decode attention ------------------------------------------ *
 * launch_attention (kernels.h:38-47, kernels.cu:846-876).  Same arguments.
 * caches [max_context][kv_heads][head_dim] fp16, positions 0..position
 * inclusive.  `scores` (heads*max_context floats, as the reference sizes it,
 * qwen_model.cpp:233) is used as the split-KV workspace when large enough;
 * otherwise the library keeps its own per-device workspace (allocated on the
 * first call that needs it, kept until citlali_hip_release_workspace()).
 * It no longer receives the raw scores.  head_dim 64 or 128, heads/kv_heads
 * between 1 and 8.  The split of the positions over workgroups is planned
 * for citlali_hip_attention_plan_length(position + 1, max_context), so all
 * steps of one such length run the same launches. */
int citlali_hip_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* scores,
                          uint16_t* out, int position, int max_context, int heads, int kv_heads, int head_dim);

/* Attention that allocates nothing.  No counterpart in the reference: for
 * callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments and results as citlali_hip_attention (bit for bit, same
 * launches) without `scores`: the split-KV partials go to a file-scope
 * device array of the library, CITLALI_NOALLOC_SCRATCH_BYTES per GPU, whose
 * device address citlali_hip_init resolves (or the first call on a GPU that
 * init did not select); the GPU holds it until the process ends.  A plan
 * whose partials (heads * chunks * (head_dim + 4) * 4 bytes) exceed it --
 * more than 496 chunks at 64 query heads of head_dim 128; every plan of at
 * most 32 query heads fits (at most 512 chunks) -- is rejected with
 * CITLALI_ERR_INVALID before anything launches.  Every call on a GPU shares that GPU's array,
 * which keeps the last call's partials: calls that overlap on one GPU (from
 * several streams or threads) race. */
#define CITLALI_NOALLOC_SCRATCH_BYTES (16u << 20)
int citlali_hip_attention_noalloc(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                  uint16_t* out, int position, int max_context, int heads, int kv_heads,
                                  int head_dim);

/* Many independent sequences in one launch (no reference counterpart: the
 * reference decodes one sequence; per sequence the result equals
 * launch_attention).  q/out [nseq][heads][head_dim]; sequence s uses the
 * caches at k_cache + s*seq_stride (elements); positions: device int32
 * [nseq], each < max_positions_bound (a larger one is treated as
 * max_positions_bound - 1, so no read leaves the caches); workspace of
 * citlali_hip_attention_workspace_bytes() bytes (may be NULL if that is 0). */
int citlali_hip_attention_batched(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                  long long seq_stride, const int32_t* positions, int max_positions_bound,
                                  int nseq, int heads, int kv_heads, int head_dim, void* workspace,
                                  size_t workspace_bytes, uint16_t* out);
/* The length attention is planned for at `length` = position + 1 (no
 * reference counterpart): the smallest power of two >= max(length, 256),
 * at most max_context; 0 for length <= 0 or length > max_context.  A step
 * replayed with the position in device memory (citlali_hip_attention_batched
 * with nseq 1 and this max_positions_bound) equals citlali_hip_attention at
 * every position of the bucket, bit for bit. */
int citlali_hip_attention_plan_length(int length, int max_context);
/* Workspace bytes that hold the split-KV partials of the plan for every
 * bound in [1, max_positions_bound] (no reference counterpart; the
 * reference's scores buffer is heads*max_context floats): the planned chunk
 * count is not monotone in the length, so a buffer sized for the longest
 * length alone can be too small for a shorter bucket.  0 when no length up
 * to the bound splits. */
size_t citlali_hip_attention_workspace_bytes(int max_positions_bound, int nseq, int heads, int kv_heads,
                                             int head_dim);
/* The plan citlali_hip_attention_batched makes for this bound (and
 * citlali_hip_attention for bound = its plan length): positions per
 * workgroup and chunks of the longest sequence (no reference counterpart;
 * for tests and sizing). */
int citlali_hip_attention_plan_info(int max_positions_bound, int nseq, int heads, int kv_heads, int head_dim,
                                    int* chunk, int* n_splits);
int citlali_hip_release_workspace(void);

/* citlali_hip_qk_norm_rope_store (or its _at form) followed by
 * citlali_hip_attention (or citlali_hip_attention_batched with nseq 1 and
 * max_positions_bound plan_length) in one launch, with the same results bit
 * for bit: q is the q GEMV's output (read only, not updated), k / v the
 * step's k and v; the step's k (normed, roped) and v are stored into the
 * caches at the position and attention reads them.  The position is
 * *position_at when that is not NULL (then plan_length is the bucket, and a
 * position at or beyond it writes nothing), else `position`.  workspace:
 * citlali_hip_attention_workspace_bytes(plan length) bytes.  No reference
 * counterpart (qwen_model.cpp:315-338 makes these separate launches);
 * CITLALI_ERR_UNSUPPORTED unless head_dim is 128 with 2..8 query heads per
 * kv head. */
int citlali_hip_qk_norm_rope_store_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                             const uint16_t* q_norm, const uint16_t* k_norm, int heads,
                                             int kv_heads, int head_dim, int position, const int32_t* position_at,
                                             int plan_length, int max_context, float theta, float eps,
                                             uint16_t* k_cache, uint16_t* v_cache, void* workspace,
                                             size_t workspace_bytes, uint16_t* out);

/* launch_store_kv (kernels.h:36, kernels.cu:829-843): the cache layout
 * contract, cache[position*kv_size + i] = k[i]. */
int citlali_hip_store_kv(const uint16_t* k, const uint16_t* v, uint16_t* k_cache, uint16_t* v_cache, int position,
                         int kv_size);

/* ---- load-time dequant on the device ------------------------------------- *
 * dequant_q4_k / dequant_q6_k of weight_loader.cpp:147-323 (host rule
 * rounding, bit-exact); `count` values from ceil(count/256) blocks. */
int citlali_hip_dequant_q4k_f16(const uint8_t* w, uint64_t count, uint16_t* out);
int citlali_hip_dequant_q6k_f16(const uint8_t* w, uint64_t count, uint16_t* out);

/* ---- the rest of forward_token (kernels.h:10-36) -------------------------- */
int citlali_hip_embed(const uint16_t* table, int32_t token_id, uint16_t* out, int hidden);   /* kernels.h:10 */
int citlali_hip_copy(const uint16_t* in, uint16_t* out, int n);                              /* kernels.h:12 */
int citlali_hip_add_inplace(uint16_t* target, const uint16_t* delta, int n);                 /* kernels.h:14 */
int citlali_hip_add_bias_inplace(uint16_t* target, const uint16_t* bias, int n);             /* kernels.h:16 */
int citlali_hip_rms_norm(const uint16_t* in, const uint16_t* w, uint16_t* out, int n, float eps); /* kernels.h:18 */
int citlali_hip_rms_norm_heads(const uint16_t* in, const uint16_t* w, uint16_t* out, int heads, int head_dim,
                               float eps);                                                    /* kernels.h:20 */
int citlali_hip_matvec_fp16(const uint16_t* w, const uint16_t* x, uint16_t* y, int in_features,
                            int out_features);                                                /* kernels.h:22 */
int citlali_hip_matvec_fp16_to_float(const uint16_t* w, const uint16_t* x, float* y, int in_features,
                                     int out_features);                                       /* kernels.h:24 */
int citlali_hip_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, int n);      /* kernels.h:34 */
int citlali_hip_rope(uint16_t* data, int heads, int head_dim, int position, float theta);    /* kernels.h:35 */

/* Greedy sampling on the device: index of the first greatest finite logit
 * (0 if none; -0.0 equals +0.0), written to device int32 *out_index.
 * Replaces the host loop of sample_greedy_from_logits (qwen_model.cpp:
 * 448-465).  Uses a per-device partials table in the library: argmax calls
 * that overlap on one device (several streams) race. */
int citlali_hip_argmax(const float* logits, int n, int32_t* out_index);

/* ---- replayable decode steps (no reference counterpart) ------------------ *
 * A decode step whose inputs live in device memory can be captured once in
 * a HIP graph and replayed per token without host synchronisation.  The
 * decode state is device int32 state[4] = {token, position, step, 0},
 * 16-byte aligned.
 * citlali_hip_argmax_advance: citlali_hip_argmax of logits, then
 *   tokens[step] = pick (when step < capacity), token = pick, position += 1,
 *   step += 1.
 * citlali_hip_embed_q6k_at / citlali_hip_embed_at: embed_q6k / embed with the
 *   token read from `token` (device); a token outside [0, vocab) gives a
 *   zero row.
 * citlali_hip_qk_norm_rope_store_at: qk_norm_rope_store with the position
 *   read from `position` (device); a position outside [0, max_positions)
 *   writes nothing to the caches. */
int citlali_hip_argmax_advance(const float* logits, int n, int32_t* state, int32_t* tokens, int capacity);
int citlali_hip_embed_q6k_at(const uint8_t* table, const int32_t* token, int vocab, uint16_t* out, int hidden);
int citlali_hip_embed_at(const uint16_t* table, const int32_t* token, int vocab, uint16_t* out, int hidden);
int citlali_hip_qk_norm_rope_store_at(uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                                      const uint16_t* k_norm, int heads, int kv_heads, int head_dim,
                                      const int32_t* position, int max_positions, float theta, float eps,
                                      uint16_t* k_cache, uint16_t* v_cache);
/* Streams and graphs.  citlali_hip_graph_begin starts capturing the launches
 * the calling thread makes on the library stream (which must not be the null
 * stream); citlali_hip_graph_end stops the capture (also after a failed
 * launch) and returns an executable graph, replayed on the library stream by
 * citlali_hip_graph_launch.  Nothing may allocate during a capture (the
 * attention workspace must come from the caller).  A graph keeps the
 * pointers and scalars it captured. */
int citlali_hip_stream_create(void** stream);
int citlali_hip_stream_destroy(void* stream);
int citlali_hip_graph_begin(void);
int citlali_hip_graph_end(void** graph);
int citlali_hip_graph_launch(void* graph);
int citlali_hip_graph_destroy(void* graph);

/* ---- timing (bench and tests) --------------------------------------------- */
/* Reads `bytes` (16-byte multiple) of a device buffer once, as fast as the
 * memory system allows: the measured HBM read ceiling.  `sink`: 4 bytes. */
int citlali_hip_stream_read(const void* buf, size_t bytes, void* sink);
/* ---- fused forward_token steps (no reference counterpart) ---------------- *
 * Each equals the sequence of reference launches it names, bit for bit (same
 * fp16 store points and reduction order); QwenModel uses them to cut the
 * launches per layer.                                                       */
/* launch_add_inplace(x, delta) then launch_rms_norm(x, w, out) */
int citlali_hip_add_rms_norm(uint16_t* x, const uint16_t* delta, const uint16_t* w, uint16_t* out, int n, float eps);
/* launch_rms_norm_heads on q and k (skipped for a NULL weight), launch_rope
 * on q and k, launch_store_kv(k, v) -- q rewritten in place, k and v written
 * to the caches at `position`.  head_dim even and <= 128. */
int citlali_hip_qk_norm_rope_store(uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                                   const uint16_t* k_norm, int heads, int kv_heads, int head_dim, int position,
                                   float theta, float eps, uint16_t* k_cache, uint16_t* v_cache);
/* GEMV weight types of the grouped / fused entry points below: GGUF type
 * 12 = Q4_K or 14 = Q6_K (KeepQuantized blocks; Q4_K 16-byte, Q6_K 4-byte
 * aligned), or 1 = F16 (DequantizeToFp16 rows, the weight pointer to the
 * fp16 values, 16-byte aligned; the results equal citlali_hip_matvec_fp16 /
 * _to_float bit for bit).
 *
 * LinearBackend::forward for ffn_gate and ffn_up (both of GGUF type
 * `gguf_type`) then launch_swiglu.  Returns
 * CITLALI_ERR_UNSUPPORTED, launching nothing, for in_features other than
 * 1024, 2048, 2560, 3072, 4096, 5120 or 8192 -- then use the separate
 * launches. */
int citlali_hip_matvec_gate_up_swiglu(int gguf_type, const uint8_t* w_gate, const uint8_t* w_up, const uint16_t* x,
                                      uint16_t* act, int in_features, int out_features);
/* LinearBackend::forward (linear_backend.cpp:17-61) for `count` (1..3)
 * weights that read the same input -- attn_q, attn_k and attn_v of one
 * layer (qwen_model.cpp:315-321) -- in one launch.  gguf_types[i] is 12 =
 * Q4_K, 14 = Q6_K or 1 = F16 (all or none), outputs[i] receives
 * out_features[i] fp16 values: the results of the separate
 * citlali_hip_matvec_q4k / _q6k / _fp16 calls bit for bit.  Outputs must
 * not overlap each other or x.  Returns CITLALI_ERR_UNSUPPORTED, launching
 * nothing, for in_features other than 1024, 2048, 2560, 3072, 4096, 5120,
 * 6144, 8192, 9728, 12288 or 16384, or F16 mixed with quantized types --
 * then use the separate launches. */
int citlali_hip_matvec_group(int count, const int* gguf_types, const uint8_t* const* weights, const uint16_t* x,
                             uint16_t* const* outputs, const int* out_features, int in_features);

/* GEMVs whose input is a residual add + RMSNorm (no reference counterpart):
 * the GEMV reads fp16(s * rsqrt(mean(s^2) + eps) * weight) with
 * s = fp16(x + delta) (s = x when delta is NULL); when sum_out is not NULL
 * it receives s.  The results equal citlali_hip_add_rms_norm(x, delta,
 * weight, tmp) followed by the plain GEMV on tmp, bit for bit (same
 * reduction order), without the separate launch: the reference's
 * add_inplace + rms_norm before attn_q/k/v, ffn_gate/up and the output
 * (qwen_model.cpp:306, 340-341, 372, 385).  weight, delta and sum_out
 * 16-byte aligned; sum_out must not be x or delta.  in_features 1024,
 * 2048, 2560, 3072, 4096, 5120, 6144, 8192, 9728, 12288 or 16384 (gate_up:
 * 1024, 2048, 2560, 3072, 4096, 5120 or 8192), else CITLALI_ERR_UNSUPPORTED
 * with nothing launched. */
typedef struct citlali_hip_norm {
    const uint16_t* delta;
    const uint16_t* weight;
    uint16_t* sum_out;
    float eps;
} citlali_hip_norm;
int citlali_hip_matvec_group_norm(int count, const int* gguf_types, const uint8_t* const* weights, const uint16_t* x,
                                  const citlali_hip_norm* norm, uint16_t* const* outputs, const int* out_features,
                                  int in_features);
int citlali_hip_matvec_gate_up_swiglu_norm(int gguf_type, const uint8_t* w_gate, const uint8_t* w_up,
                                           const uint16_t* x, const citlali_hip_norm* norm, uint16_t* act,
                                           int in_features, int out_features);
/* gguf_type 12 / 14 / 1; y fp16 (f32_out 0) or fp32 (f32_out 1) */
int citlali_hip_matvec_norm(int gguf_type, const uint8_t* w, const uint16_t* x, const citlali_hip_norm* norm,
                            void* y, int f32_out, int in_features, int out_features);

/* Kernel timing (no reference counterpart; for benchmarks): while armed with
 * two events of citlali_hip_event_create, the first kernel the calling thread
 * launches records `start` when it begins and every kernel records `stop`
 * when it ends, stamped from the dispatch itself (hipExtLaunchKernel), so
 * citlali_hip_event_elapsed_ms(start, stop) is the kernels' own time.  Arm
 * before a call, disarm with (NULL, NULL) after it. */
int citlali_hip_set_kernel_timing(void* start, void* stop);
/* Per-dispatch kernel timing (no reference counterpart; for benchmarks):
 * while armed with n pairs of events (1 <= n <= CITLALI_MAX_TIMED_DISPATCHES),
 * the i-th kernel the calling thread launches, i < n, records starts[i] when
 * it begins and stops[i] when it ends, stamped from the dispatch itself, so a
 * call of several kernels gives each kernel's own time without the gaps
 * between them.  citlali_hip_dispatch_timing_count gives how many kernels
 * were launched since arming (those past n are not stamped), also after
 * disarming with (NULL, NULL, 0).  Not together with
 * citlali_hip_set_kernel_timing, nor during graph capture. */
#define CITLALI_MAX_TIMED_DISPATCHES 64
int citlali_hip_set_dispatch_timing(void* const* starts, void* const* stops, int n);
int citlali_hip_dispatch_timing_count(int* count);
int citlali_hip_event_create(void** event);
int citlali_hip_event_record(void* event);                  /* on the current stream */
int citlali_hip_event_synchronize(void* event);
int citlali_hip_event_elapsed_ms(void* start, void* stop, float* ms);
int citlali_hip_event_destroy(void* event);

#ifdef __cplusplus
}
#endif

#endif /* CITLALI_HIP_H */
