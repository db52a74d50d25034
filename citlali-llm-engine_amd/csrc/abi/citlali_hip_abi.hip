// citlali_hip_abi.hip -- the extern "C" boundary (include/citlali_hip.h).
//
// Validates arguments on the host (before anything touches the GPU), then
// calls the gfx950 launchers.  Errors are reported as status codes plus a
// thread-local message.
#include "../kernels/launch.hpp"
#include "citlali_hip.h"

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <mutex>
#include <thread>
#include <vector>

#define CITLALI_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

thread_local char g_err[512] = "";
hipStream_t g_stream = nullptr;

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(hipError_t e, const char* expr, const char* file, int line) {
    if (e == hipSuccess) return CITLALI_OK;
    return fail(CITLALI_ERR_HIP, "HIP error at %s:%d for %s: %s", file, line, expr, hipGetErrorString(e));
}
#define HIP_TRY(expr)                                                          \
    do {                                                                       \
        const int _st = hip_status((expr), #expr, __FILE__, __LINE__);         \
        if (_st != CITLALI_OK) return _st;                                     \
    } while (0)

#define REQUIRE(cond, ...)                                  \
    do {                                                    \
        if (!(cond)) return fail(CITLALI_ERR_INVALID, __VA_ARGS__); \
    } while (0)

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int check_matvec(const char* who, const void* w, const void* x, const void* y, int in_f, int out_f, uintptr_t walign,
                 uintptr_t yalign) {
    REQUIRE(w && x && y, "%s received a null buffer", who);
    REQUIRE(in_f > 0 && out_f > 0, "%s: in_features (%d) and out_features (%d) must be positive", who, in_f, out_f);
    REQUIRE(in_f % 256 == 0, "%s: in_features (%d) is not a multiple of the 256-value super-block", who, in_f);
    REQUIRE(in_f <= CITLALI_MAX_IN_FEATURES, "%s: in_features (%d) exceeds %d", who, in_f, CITLALI_MAX_IN_FEATURES);
    REQUIRE(aligned(w, walign), "%s: weight pointer must be %d-byte aligned", who, (int)walign);
    REQUIRE(aligned(x, 16), "%s: input pointer must be 16-byte aligned", who);
    REQUIRE(aligned(y, yalign), "%s: output pointer must be %d-byte aligned", who, (int)yalign);
    return CITLALI_OK;
}

// Per-device attention workspace kept by the library for the split-KV
// partials when the caller's `scores` buffer is too small.  It grows on
// demand; launches that overlap on one device would share it.
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
constexpr int kMaxDevices = 64;
Workspace g_ws[kMaxDevices];
std::mutex g_ws_mu;

int workspace_for(size_t bytes, float** out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    REQUIRE(dev >= 0 && dev < kMaxDevices, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = g_ws[dev];
    if (w.bytes < bytes) {
        if (w.ptr) {
            // a launch queued on any stream (the library stream may have
            // changed since) may still use it
            HIP_TRY(hipDeviceSynchronize());
            HIP_TRY(hipFree(w.ptr));
        }
        w.ptr = nullptr;
        w.bytes = 0;
        HIP_TRY(hipMalloc(&w.ptr, bytes));
        w.bytes = bytes;
    }
    *out = static_cast<float*>(w.ptr);
    return CITLALI_OK;
}

constexpr int kAttnTargetBlocks = 256;   // one workgroup per CU

// ---- scratch of the entry point that allocates nothing ----------------------
// citlali_hip_attention_noalloc keeps its split-KV partials in this array:
// one copy per GPU, held from the library's first use on that GPU until the
// process ends.  In host code `scratch` names a host-side stand-in, not
// device memory; the device address of each GPU's copy comes from
// hipGetSymbolAddress with that GPU current, and only that address is given
// to kernels.
constexpr size_t kScratchBytes = CITLALI_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
void* g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// This device's copy of `scratch` (the current device), resolved once.
int scratch_for_current_device(void** out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    REQUIRE(dev >= 0 && dev < kMaxDevices, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        REQUIRE(p != nullptr && aligned(p, 256), "scratch: no device address for device %d", dev);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return CITLALI_OK;
}

// The arguments of a single-sequence decode attention at `position`
// (citlali_hip_attention and its no-allocation form).
citlali::hip::AttnArgs scalar_attention_args(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                               int position, int heads, int kv_heads, int head_dim) {
    citlali::hip::AttnArgs a{};
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.seq_stride = 0;
    a.positions = nullptr;
    a.position = position;
    a.max_len = position + 1;
    a.nseq = 1;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.out = out;
    return a;
}

}  // namespace

namespace citlali::hip {
KernelTiming& kernel_timing() {
    thread_local KernelTiming t;
    return t;
}
}  // namespace citlali::hip

using namespace citlali::hip;

// ---------------------------------------------------------------- runtime
CITLALI_EXPORT const char* citlali_hip_last_error(void) { return g_err; }
CITLALI_EXPORT int citlali_hip_abi_version(void) { return CITLALI_HIP_ABI_VERSION; }

CITLALI_EXPORT int citlali_hip_init(int device) {
    REQUIRE(device >= 0, "device index must be non-negative");
    HIP_TRY(hipSetDevice(device));
    void* s = nullptr;   // this device's no-allocation scratch, resolved at set-up
    return scratch_for_current_device(&s);
}

CITLALI_EXPORT int citlali_hip_device_count(int* count) {
    REQUIRE(count, "null output pointer");
    HIP_TRY(hipGetDeviceCount(count));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_set_stream(void* stream) {
    g_stream = static_cast<hipStream_t>(stream);
    return CITLALI_OK;
}
CITLALI_EXPORT void* citlali_hip_get_stream(void) { return g_stream; }

CITLALI_EXPORT int citlali_hip_synchronize(void) {
    HIP_TRY(hipStreamSynchronize(g_stream));
    HIP_TRY(hipGetLastError());
    return CITLALI_OK;
}

// ---------------------------------------------------------------- memory
CITLALI_EXPORT int citlali_hip_malloc(void** ptr, size_t bytes) {
    REQUIRE(ptr, "null output pointer");
    *ptr = nullptr;
    if (bytes == 0) return CITLALI_OK;
    HIP_TRY(hipMalloc(ptr, bytes));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_free(void* ptr) {
    if (ptr) HIP_TRY(hipFree(ptr));
    return CITLALI_OK;
}

namespace {
// Large host -> device copies (weight uploads, WeightLoader) go through two
// pinned staging buffers: host threads copy the next piece of the (pageable)
// source into one buffer while the DMA engine moves the other, on the
// library stream so the copy stays ordered with the launches.  Each device's
// buffers (2 x kStageBytes of pinned host memory) are allocated on first use
// and kept until the process ends; copies through them are serialised.
constexpr size_t kStageBytes = (size_t)8 << 20;
constexpr size_t kStageMin = (size_t)8 << 20;   // smaller copies: one pageable hipMemcpyAsync
struct Staging {
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool failed = false;   // pinned allocation refused: stay on the pageable path
};
Staging g_stage[kMaxDevices];
std::mutex g_stage_mu;

// memcpy split over up to 8 host threads (page-aligned pieces of >= 1 MB)
void parallel_copy(void* dst, const void* src, size_t n) {
    const unsigned hw = std::thread::hardware_concurrency();
    const size_t threads = std::min<size_t>(std::min<size_t>(8, hw ? hw : 1), n >> 20);
    if (threads <= 1) {
        std::memcpy(dst, src, n);
        return;
    }
    const size_t per = (n / threads + 4095) & ~(size_t)4095;
    std::vector<std::thread> pool;
    for (size_t off = per; off < n; off += per) {
        const size_t len = std::min(per, n - off);
        pool.emplace_back([=] { std::memcpy(static_cast<char*>(dst) + off, static_cast<const char*>(src) + off, len); });
    }
    std::memcpy(dst, src, std::min(per, n));
    for (auto& t : pool) t.join();
}

bool staging_ready(Staging& s) {
    if (s.buf[0]) return true;
    if (s.failed) return false;
    for (int i = 0; i < 2; ++i) {
        if (hipHostMalloc(&s.buf[i], kStageBytes, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&s.done[i], hipEventDisableTiming) != hipSuccess) {
            s.failed = true;
            (void)hipGetLastError();
            return false;
        }
    }
    return true;
}
}  // namespace

CITLALI_EXPORT int citlali_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return CITLALI_OK;
    REQUIRE(dst && src, "copy_from_host received a null pointer");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (bytes >= kStageMin && dev >= 0 && dev < kMaxDevices) {
        std::lock_guard<std::mutex> lock(g_stage_mu);
        Staging& s = g_stage[dev];
        if (staging_ready(s)) {
            bool used[2] = {false, false};
            for (size_t off = 0, i = 0; off < bytes; off += kStageBytes, ++i) {
                const int b = (int)(i & 1);
                const size_t n = std::min(kStageBytes, bytes - off);
                if (used[b]) HIP_TRY(hipEventSynchronize(s.done[b]));   // its previous DMA is done
                parallel_copy(s.buf[b], static_cast<const char*>(src) + off, n);
                HIP_TRY(hipMemcpyAsync(static_cast<char*>(dst) + off, s.buf[b], n, hipMemcpyHostToDevice, g_stream));
                HIP_TRY(hipEventRecord(s.done[b], g_stream));
                used[b] = true;
            }
            HIP_TRY(hipStreamSynchronize(g_stream));
            return CITLALI_OK;
        }
    }
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return CITLALI_OK;
    REQUIRE(dst && src, "copy_to_host received a null pointer");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return CITLALI_OK;
    REQUIRE(dst && src, "device copy received a null pointer");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_zero(void* ptr, size_t bytes) {
    if (bytes == 0) return CITLALI_OK;
    REQUIRE(ptr, "zero received a null pointer");
    HIP_TRY(launch_fill_zero(ptr, bytes, g_stream));
    return CITLALI_OK;
}

// ---------------------------------------------------------------- GEMV
CITLALI_EXPORT int citlali_hip_matvec_q4k(const uint8_t* w, const uint16_t* x, uint16_t* y, int in_f, int out_f) {
    const int st = check_matvec("matvec_q4k", w, x, y, in_f, out_f, 16, 2);
    if (st) return st;
    HIP_TRY(launch_matvec_q4k(w, x, y, false, in_f, out_f, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_matvec_q4k_to_float(const uint8_t* w, const uint16_t* x, float* y, int in_f,
                                                   int out_f) {
    const int st = check_matvec("matvec_q4k_to_float", w, x, y, in_f, out_f, 16, 4);
    if (st) return st;
    HIP_TRY(launch_matvec_q4k(w, x, y, true, in_f, out_f, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_matvec_q6k(const uint8_t* w, const uint16_t* x, uint16_t* y, int in_f, int out_f) {
    const int st = check_matvec("matvec_q6k", w, x, y, in_f, out_f, 4, 2);
    if (st) return st;
    HIP_TRY(launch_matvec_q6k(w, x, y, false, in_f, out_f, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_matvec_q6k_to_float(const uint8_t* w, const uint16_t* x, float* y, int in_f,
                                                   int out_f) {
    const int st = check_matvec("matvec_q6k_to_float", w, x, y, in_f, out_f, 4, 4);
    if (st) return st;
    HIP_TRY(launch_matvec_q6k(w, x, y, true, in_f, out_f, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_embed_q6k(const uint8_t* table, int32_t token_id, uint16_t* out, int hidden) {
    REQUIRE(table && out, "embed_q6k received a null buffer");
    REQUIRE(token_id >= 0, "token id out of vocab range");
    REQUIRE(hidden > 0 && hidden % 256 == 0, "embed_q6k: hidden (%d) must be a positive multiple of 256", hidden);
    HIP_TRY(launch_embed_q6k(table, token_id, nullptr, 0, out, hidden, g_stream));
    return CITLALI_OK;
}

// ---------------------------------------------------------------- attention
static int check_attn_shape(int heads, int kv_heads, int head_dim) {
    REQUIRE(heads > 0 && kv_heads > 0, "attention: heads and kv_heads must be positive");
    REQUIRE(heads % kv_heads == 0, "attention head_count must be divisible by head_count_kv");
    if (!attention_supported(head_dim, heads / kv_heads))
        return fail(CITLALI_ERR_UNSUPPORTED,
                    "attention: head_dim %d with %d query heads per kv head is not built (head_dim 64/128, group 1..8)",
                    head_dim, heads / kv_heads);
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                         float* scores, uint16_t* out, int position, int max_context, int heads,
                                         int kv_heads, int head_dim) {
    REQUIRE(q && k_cache && v_cache && out, "attention received a null buffer");
    REQUIRE(position >= 0 && position < max_context, "position exceeds max_context");
    int st = check_attn_shape(heads, kv_heads, head_dim);
    if (st) return st;
    REQUIRE(aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16), "attention: q and caches must be 16-byte aligned");

    AttnArgs a = scalar_attention_args(q, k_cache, v_cache, out, position, heads, kv_heads, head_dim);
    // planned for the length's bucket, so every step of a bucket launches the
    // same kernels (as a captured step with the position in device memory)
    const AttnPlan p = plan_attention(attention_plan_length(position + 1, max_context), 1, kv_heads, heads, head_dim,
                                      kAttnTargetBlocks);
    const size_t need = attention_workspace_bytes(p, 1, heads, head_dim);
    const size_t have = scores ? (size_t)heads * (size_t)max_context * sizeof(float) : 0;
    if (need == 0) {
        a.workspace = nullptr;
    } else if (need <= have && aligned(scores, 16)) {
        a.workspace = scores;
    } else {
        st = workspace_for(need, &a.workspace);
        if (st) return st;
    }
    HIP_TRY(launch_attention(a, p, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_attention_noalloc(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                                 uint16_t* out, int position, int max_context, int heads,
                                                 int kv_heads, int head_dim) {
    REQUIRE(q && k_cache && v_cache && out, "attention_noalloc received a null buffer");
    REQUIRE(position >= 0 && position < max_context, "position exceeds max_context");
    int st = check_attn_shape(heads, kv_heads, head_dim);
    if (st) return st;
    REQUIRE(aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16),
            "attention_noalloc: q and caches must be 16-byte aligned");
    AttnArgs a = scalar_attention_args(q, k_cache, v_cache, out, position, heads, kv_heads, head_dim);
    // the plan of citlali_hip_attention, so the same kernels and results
    const AttnPlan p = plan_attention(attention_plan_length(position + 1, max_context), 1, kv_heads, heads, head_dim,
                                      kAttnTargetBlocks);
    const size_t need = attention_workspace_bytes(p, 1, heads, head_dim);
    REQUIRE(need <= kScratchBytes,
            "attention_noalloc: the split partials of %d chunks x %d heads need %zu bytes, more than the %zu-byte "
            "scratch (CITLALI_NOALLOC_SCRATCH_BYTES)",
            p.n_splits, heads, need, kScratchBytes);
    a.workspace = nullptr;
    if (need > 0) {
        void* s = nullptr;
        st = scratch_for_current_device(&s);
        if (st) return st;
        a.workspace = static_cast<float*>(s);
    }
    HIP_TRY(launch_attention(a, p, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_attention_plan_length(int length, int max_context) {
    if (length <= 0 || max_context < length) return 0;
    return attention_plan_length(length, max_context);
}

CITLALI_EXPORT size_t citlali_hip_attention_workspace_bytes(int max_positions_bound, int nseq, int heads,
                                                            int kv_heads, int head_dim) {
    if (max_positions_bound <= 0 || nseq <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads) return 0;
    return attention_workspace_bound(max_positions_bound, nseq, kv_heads, heads, head_dim, kAttnTargetBlocks);
}

CITLALI_EXPORT int citlali_hip_attention_plan_info(int max_positions_bound, int nseq, int heads, int kv_heads,
                                                   int head_dim, int* chunk, int* n_splits) {
    REQUIRE(chunk && n_splits, "attention_plan_info: null output pointer");
    REQUIRE(max_positions_bound > 0 && nseq > 0, "attention_plan_info: bound and nseq must be positive");
    const int st = check_attn_shape(heads, kv_heads, head_dim);
    if (st) return st;
    const AttnPlan p = plan_attention(max_positions_bound, nseq, kv_heads, heads, head_dim, kAttnTargetBlocks);
    *chunk = p.chunk;
    *n_splits = p.n_splits;
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_attention_batched(const uint16_t* q, const uint16_t* k_cache,
                                                 const uint16_t* v_cache, long long seq_stride,
                                                 const int32_t* positions, int max_positions_bound, int nseq,
                                                 int heads, int kv_heads, int head_dim, void* workspace,
                                                 size_t workspace_bytes, uint16_t* out) {
    REQUIRE(q && k_cache && v_cache && out && positions, "attention_batched received a null buffer");
    REQUIRE(nseq > 0, "attention_batched: nseq must be positive");
    REQUIRE(max_positions_bound > 0, "attention_batched: max_positions_bound must be positive");
    REQUIRE(seq_stride >= 0, "attention_batched: negative sequence stride");
    const int st = check_attn_shape(heads, kv_heads, head_dim);
    if (st) return st;
    REQUIRE(aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16) && (seq_stride % 8) == 0,
            "attention_batched: q, caches and sequence stride must be 16-byte aligned");
    const AttnPlan p = plan_attention(max_positions_bound, nseq, kv_heads, heads, head_dim, kAttnTargetBlocks);
    const size_t need = attention_workspace_bytes(p, nseq, heads, head_dim);
    REQUIRE(workspace_bytes >= need && (need == 0 || (workspace && aligned(workspace, 16))),
            "attention_batched: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    AttnArgs a{};
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.seq_stride = seq_stride;
    a.positions = positions;
    a.position = 0;
    a.max_len = max_positions_bound;
    a.nseq = nseq;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.workspace = static_cast<float*>(workspace);
    a.out = out;
    HIP_TRY(launch_attention(a, p, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_release_workspace(void) {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    int cur = 0;
    HIP_TRY(hipGetDevice(&cur));
    int st = CITLALI_OK;
    for (int d = 0; d < kMaxDevices && st == CITLALI_OK; ++d) {
        Workspace& w = g_ws[d];
        if (!w.ptr) continue;
        st = hip_status(hipSetDevice(d), "hipSetDevice(d)", __FILE__, __LINE__);
        if (st == CITLALI_OK) st = hip_status(hipDeviceSynchronize(), "hipDeviceSynchronize()", __FILE__, __LINE__);
        if (st == CITLALI_OK) st = hip_status(hipFree(w.ptr), "hipFree(w.ptr)", __FILE__, __LINE__);
        if (st == CITLALI_OK) {
            w.ptr = nullptr;
            w.bytes = 0;
        }
    }
    const int st2 = hip_status(hipSetDevice(cur), "hipSetDevice(cur)", __FILE__, __LINE__);
    return st != CITLALI_OK ? st : st2;
}

CITLALI_EXPORT int citlali_hip_store_kv(const uint16_t* k, const uint16_t* v, uint16_t* kc, uint16_t* vc,
                                        int position, int kv_size) {
    REQUIRE(k && v && kc && vc, "store_kv received a null buffer");
    REQUIRE(position >= 0 && kv_size > 0, "store_kv: bad position (%d) or kv_size (%d)", position, kv_size);
    HIP_TRY(launch_store_kv(k, v, kc, vc, position, kv_size, g_stream));
    return CITLALI_OK;
}

// ---------------------------------------------------------------- dequant
CITLALI_EXPORT int citlali_hip_dequant_q4k_f16(const uint8_t* w, uint64_t count, uint16_t* out) {
    REQUIRE(w && out, "dequant_q4k received a null buffer");
    if (count == 0) return CITLALI_OK;
    HIP_TRY(launch_dequant_q4k_f16(w, count, out, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_dequant_q6k_f16(const uint8_t* w, uint64_t count, uint16_t* out) {
    REQUIRE(w && out, "dequant_q6k received a null buffer");
    if (count == 0) return CITLALI_OK;
    HIP_TRY(launch_dequant_q6k_f16(w, count, out, g_stream));
    return CITLALI_OK;
}

// ---------------------------------------------------------------- rest of the step
CITLALI_EXPORT int citlali_hip_embed(const uint16_t* table, int32_t token_id, uint16_t* out, int hidden) {
    REQUIRE(table && out, "embed received a null buffer");
    REQUIRE(token_id >= 0 && hidden > 0, "embed: bad token id or hidden size");
    HIP_TRY(launch_embed_f16(table, token_id, nullptr, 0, out, hidden, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_copy(const uint16_t* in, uint16_t* out, int n) {
    REQUIRE(in && out && n > 0, "copy: bad arguments");
    HIP_TRY(launch_copy(in, out, n, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_add_inplace(uint16_t* t, const uint16_t* d, int n) {
    REQUIRE(t && d && n > 0, "add_inplace: bad arguments");
    HIP_TRY(launch_add_inplace(t, d, n, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_add_bias_inplace(uint16_t* t, const uint16_t* b, int n) {
    REQUIRE(t && b && n > 0, "add_bias_inplace: bad arguments");
    HIP_TRY(launch_add_inplace(t, b, n, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_rms_norm(const uint16_t* in, const uint16_t* w, uint16_t* out, int n, float eps) {
    REQUIRE(in && w && out && n > 0, "rms_norm: bad arguments");
    HIP_TRY(launch_rms_norm(in, w, out, n, eps, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_rms_norm_heads(const uint16_t* in, const uint16_t* w, uint16_t* out, int heads,
                                              int head_dim, float eps) {
    REQUIRE(in && w && out && heads > 0 && head_dim > 0, "rms_norm_heads: bad arguments");
    HIP_TRY(launch_rms_norm_heads(in, w, out, heads, head_dim, eps, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_matvec_fp16(const uint16_t* w, const uint16_t* x, uint16_t* y, int in_f, int out_f) {
    REQUIRE(w && x && y && in_f > 0 && out_f > 0, "matvec_fp16: bad arguments");
    REQUIRE((in_f % 8) != 0 || (aligned(w, 16) && aligned(x, 16)), "matvec_fp16: buffers must be 16-byte aligned");
    HIP_TRY(launch_matvec_f16(w, x, y, false, in_f, out_f, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_matvec_fp16_to_float(const uint16_t* w, const uint16_t* x, float* y, int in_f,
                                                    int out_f) {
    REQUIRE(w && x && y && in_f > 0 && out_f > 0, "matvec_fp16_to_float: bad arguments");
    REQUIRE((in_f % 8) != 0 || (aligned(w, 16) && aligned(x, 16)), "matvec_fp16: buffers must be 16-byte aligned");
    HIP_TRY(launch_matvec_f16(w, x, y, true, in_f, out_f, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_swiglu(const uint16_t* g, const uint16_t* u, uint16_t* out, int n) {
    REQUIRE(g && u && out && n > 0, "swiglu: bad arguments");
    HIP_TRY(launch_swiglu(g, u, out, n, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_rope(uint16_t* data, int heads, int head_dim, int position, float theta) {
    REQUIRE(data && heads > 0 && head_dim > 0 && head_dim % 2 == 0 && head_dim <= 2048, "rope: bad arguments");
    HIP_TRY(launch_rope(data, heads, head_dim, position, theta, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_argmax(const float* logits, int n, int32_t* out_index) {
    REQUIRE(logits && out_index && n > 0, "argmax: bad arguments");
    HIP_TRY(launch_argmax(logits, n, out_index, nullptr, nullptr, 0, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_argmax_advance(const float* logits, int n, int32_t* state, int32_t* tokens,
                                              int capacity) {
    REQUIRE(logits && state && n > 0, "argmax_advance: bad arguments");
    REQUIRE(capacity >= 0 && (capacity == 0 || tokens), "argmax_advance: bad token array");
    REQUIRE(aligned(state, 16), "argmax_advance: state must be 16-byte aligned");
    HIP_TRY(launch_argmax(logits, n, nullptr, state, tokens, capacity, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_embed_q6k_at(const uint8_t* table, const int32_t* token, int vocab, uint16_t* out,
                                            int hidden) {
    REQUIRE(table && token && out, "embed_q6k_at received a null buffer");
    REQUIRE(vocab > 0, "embed_q6k_at: vocab must be positive");
    REQUIRE(hidden > 0 && hidden % 256 == 0, "embed_q6k_at: hidden (%d) must be a positive multiple of 256", hidden);
    HIP_TRY(launch_embed_q6k(table, 0, token, vocab, out, hidden, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_embed_at(const uint16_t* table, const int32_t* token, int vocab, uint16_t* out,
                                        int hidden) {
    REQUIRE(table && token && out, "embed_at received a null buffer");
    REQUIRE(vocab > 0 && hidden > 0, "embed_at: bad vocab or hidden size");
    HIP_TRY(launch_embed_f16(table, 0, token, vocab, out, hidden, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_stream_read(const void* buf, size_t bytes, void* sink) {
    REQUIRE(buf && sink && aligned(buf, 16) && aligned(sink, 4), "stream_read: bad arguments");
    HIP_TRY(launch_stream_read(buf, bytes, static_cast<uint32_t*>(sink), g_stream));
    return CITLALI_OK;
}

// ---------------------------------------------------------------- events
CITLALI_EXPORT int citlali_hip_add_rms_norm(uint16_t* x, const uint16_t* delta, const uint16_t* w, uint16_t* out,
                                            int n, float eps) {
    REQUIRE(x && delta && w && out && n > 0, "add_rms_norm: bad arguments");
    HIP_TRY(launch_add_rms_norm(x, delta, w, out, n, eps, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_qk_norm_rope_store(uint16_t* q, const uint16_t* k, const uint16_t* v,
                                                  const uint16_t* q_norm, const uint16_t* k_norm, int heads,
                                                  int kv_heads, int head_dim, int position, float theta, float eps,
                                                  uint16_t* k_cache, uint16_t* v_cache) {
    REQUIRE(q && k && v && k_cache && v_cache, "qk_norm_rope_store received a null buffer");
    REQUIRE(heads > 0 && kv_heads > 0 && position >= 0, "qk_norm_rope_store: bad heads or position");
    REQUIRE(head_dim > 0 && head_dim <= 128 && head_dim % 2 == 0, "qk_norm_rope_store: head_dim %d not supported",
            head_dim);
    HIP_TRY(launch_qk_norm_rope_store(q, k, v, q_norm, k_norm, heads, kv_heads, head_dim, position, nullptr, INT_MAX,
                                      theta, eps, k_cache, v_cache, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_qk_norm_rope_store_at(uint16_t* q, const uint16_t* k, const uint16_t* v,
                                                     const uint16_t* q_norm, const uint16_t* k_norm, int heads,
                                                     int kv_heads, int head_dim, const int32_t* position,
                                                     int max_positions, float theta, float eps, uint16_t* k_cache,
                                                     uint16_t* v_cache) {
    REQUIRE(q && k && v && k_cache && v_cache && position, "qk_norm_rope_store_at received a null buffer");
    REQUIRE(heads > 0 && kv_heads > 0 && max_positions > 0, "qk_norm_rope_store_at: bad heads or max_positions");
    REQUIRE(head_dim > 0 && head_dim <= 128 && head_dim % 2 == 0,
            "qk_norm_rope_store_at: head_dim %d not supported", head_dim);
    HIP_TRY(launch_qk_norm_rope_store(q, k, v, q_norm, k_norm, heads, kv_heads, head_dim, 0, position,
                                      max_positions, theta, eps, k_cache, v_cache, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_qk_norm_rope_store_attention(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm, const uint16_t* k_norm,
    int heads, int kv_heads, int head_dim, int position, const int32_t* position_at, int plan_length,
    int max_context, float theta, float eps, uint16_t* k_cache, uint16_t* v_cache, void* workspace,
    size_t workspace_bytes, uint16_t* out) {
    REQUIRE(q && k && v && k_cache && v_cache && out, "qk_norm_rope_store_attention received a null buffer");
    const int st = check_attn_shape(heads, kv_heads, head_dim);
    if (st) return st;
    const int group = heads / kv_heads;
    if (head_dim != 128 || group < 2 || group > 8)
        return fail(CITLALI_ERR_UNSUPPORTED,
                    "qk_norm_rope_store_attention: no fused kernel for head_dim %d with %d query heads per kv head",
                    head_dim, group);
    REQUIRE(aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16),
            "qk_norm_rope_store_attention: q and caches must be 16-byte aligned");
    REQUIRE(max_context > 0, "qk_norm_rope_store_attention: max_context must be positive");
    AttnArgs a{};
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.seq_stride = 0;
    a.nseq = 1;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.out = out;
    AttnPlan p{};
    if (position_at != nullptr) {
        // as qk_norm_rope_store_at + attention_batched(nseq 1, plan_length)
        REQUIRE(plan_length > 0 && plan_length <= max_context,
                "qk_norm_rope_store_attention: plan_length %d outside (0, max_context]", plan_length);
        a.positions = position_at;
        a.max_len = plan_length;
        p = plan_attention(plan_length, 1, kv_heads, heads, head_dim, kAttnTargetBlocks);
    } else {
        // as qk_norm_rope_store + attention at `position`
        REQUIRE(position >= 0 && position < max_context, "position exceeds max_context");
        a.position = position;
        a.max_len = position + 1;
        p = plan_attention(attention_plan_length(position + 1, max_context), 1, kv_heads, heads, head_dim,
                           kAttnTargetBlocks);
    }
    const size_t need = attention_workspace_bytes(p, 1, heads, head_dim);
    REQUIRE(workspace_bytes >= need && (need == 0 || (workspace && aligned(workspace, 16))),
            "qk_norm_rope_store_attention: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    a.workspace = static_cast<float*>(workspace);
    const QkPrep prep{k, v, q_norm, k_norm, k_cache, v_cache, theta, eps};
    a.prep = &prep;
    HIP_TRY(launch_attention(a, p, g_stream));
    return CITLALI_OK;
}

// ---------------------------------------------------------------- streams and graphs
CITLALI_EXPORT int citlali_hip_stream_create(void** stream) {
    REQUIRE(stream, "null output pointer");
    hipStream_t st = nullptr;
    HIP_TRY(hipStreamCreate(&st));
    *stream = st;
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_stream_destroy(void* stream) {
    REQUIRE(stream, "stream_destroy: null stream");
    REQUIRE(stream != g_stream, "stream_destroy: the stream is the library stream");
    HIP_TRY(hipStreamDestroy(static_cast<hipStream_t>(stream)));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_graph_begin(void) {
    REQUIRE(g_stream != nullptr, "graph_begin: capture needs a library stream other than the null stream");
    REQUIRE(kernel_timing().start == nullptr && kernel_timing().starts.empty(), "graph_begin: kernel timing is armed");
    HIP_TRY(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_graph_end(void** graph) {
    REQUIRE(graph, "null output pointer");
    *graph = nullptr;
    REQUIRE(g_stream != nullptr, "graph_end: no capture on the null stream");
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamEndCapture(g_stream, &g));   // ends the capture even when it failed
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HIP_TRY(e);
    *graph = exec;
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_graph_launch(void* graph) {
    REQUIRE(graph, "graph_launch: null graph");
    HIP_TRY(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_graph_destroy(void* graph) {
    REQUIRE(graph, "graph_destroy: null graph");
    HIP_TRY(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)));
    return CITLALI_OK;
}

namespace {
// Row lengths the grouped / prologue / gate-up GEMV kernels cover
bool norm_length_ok(int in_f) { return matvec_fused_length(in_f, true); }
bool group_length_ok(int in_f) { return matvec_fused_length(in_f, true); }   // hidden-sized inputs
bool gate_up_length_ok(int in_f) { return matvec_gate_up_length(in_f); }
// GEMV weight types of the grouped / fused entry points: GGUF Q4_K (12),
// Q6_K (14) and F16 (1, fp16 rows), as the kernels' kinds 4, 6, 1
bool fused_type_ok(int t) { return t == 12 || t == 14 || t == 1; }
int fused_kind(int t) { return t == 14 ? 6 : t == 1 ? 1 : 4; }
uintptr_t fused_walign(int t) { return t == 14 ? 4 : 16; }
}  // namespace

CITLALI_EXPORT int citlali_hip_matvec_gate_up_swiglu(int gguf_type, const uint8_t* w_gate, const uint8_t* w_up,
                                                     const uint16_t* x, uint16_t* act, int in_f, int out_f) {
    REQUIRE(fused_type_ok(gguf_type), "matvec_gate_up_swiglu: GGUF type %d is not Q4_K, Q6_K or F16", gguf_type);
    const uintptr_t walign = fused_walign(gguf_type);
    int st = check_matvec("matvec_gate_up_swiglu", w_gate, x, act, in_f, out_f, walign, 2);
    if (st) return st;
    REQUIRE(w_up && aligned(w_up, walign), "matvec_gate_up_swiglu: bad up weight");
    if (!gate_up_length_ok(in_f))
        return fail(CITLALI_ERR_UNSUPPORTED, "matvec_gate_up_swiglu: in_features %d has no fused kernel", in_f);
    HIP_TRY(launch_matvec_gate_up_swiglu(fused_kind(gguf_type), w_gate, w_up, x, act, in_f, out_f, nullptr,
                                         g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_matvec_group(int count, const int* gguf_types, const uint8_t* const* weights,
                                            const uint16_t* x, uint16_t* const* outputs, const int* out_features,
                                            int in_f) {
    REQUIRE(count >= 1 && count <= 3, "matvec_group: count %d is not 1, 2 or 3", count);
    REQUIRE(gguf_types && weights && outputs && out_features, "matvec_group received a null array");
    int kinds[3];
    long long rows = 0;
    int f16 = 0;
    for (int i = 0; i < count; ++i) {
        REQUIRE(fused_type_ok(gguf_types[i]), "matvec_group: GGUF type %d is not Q4_K, Q6_K or F16", gguf_types[i]);
        const int st = check_matvec("matvec_group", weights[i], x, outputs[i], in_f, out_features[i],
                                    fused_walign(gguf_types[i]), 2);
        if (st) return st;
        kinds[i] = fused_kind(gguf_types[i]);
        f16 += kinds[i] == 1;
        rows += out_features[i];
    }
    REQUIRE(rows <= INT_MAX, "matvec_group: %lld rows in total exceed INT_MAX", rows);
    if (f16 != 0 && f16 != count)
        return fail(CITLALI_ERR_UNSUPPORTED, "matvec_group: F16 and quantized weights have no grouped kernel");
    if (!group_length_ok(in_f))
        return fail(CITLALI_ERR_UNSUPPORTED, "matvec_group: in_features %d has no grouped kernel", in_f);
    HIP_TRY(launch_matvec_group(count, kinds, weights, x, outputs, out_features, in_f, nullptr, g_stream));
    return CITLALI_OK;
}

// ---------------------------------------------------------------- GEMVs with the add + RMSNorm prologue
namespace {
int check_norm(const char* who, const uint16_t* x, const citlali_hip_norm* n, int in_f, NormIn* out) {
    REQUIRE(n, "%s: null norm", who);
    REQUIRE(n->weight && aligned(n->weight, 16), "%s: norm weight must be non-null and 16-byte aligned", who);
    REQUIRE(!n->delta || aligned(n->delta, 16), "%s: delta must be 16-byte aligned", who);
    REQUIRE(!n->sum_out || aligned(n->sum_out, 16), "%s: sum_out must be 16-byte aligned", who);
    REQUIRE(!n->sum_out || (n->sum_out != x && n->sum_out != n->delta),
            "%s: sum_out must not be the input or the delta (every workgroup reads them)", who);
    *out = NormIn{n->delta, n->weight, n->sum_out, n->eps};
    (void)in_f;
    return CITLALI_OK;
}
}  // namespace

CITLALI_EXPORT int citlali_hip_matvec_group_norm(int count, const int* gguf_types, const uint8_t* const* weights,
                                                 const uint16_t* x, const citlali_hip_norm* norm,
                                                 uint16_t* const* outputs, const int* out_features, int in_f) {
    REQUIRE(count >= 1 && count <= 3, "matvec_group_norm: count %d is not 1, 2 or 3", count);
    REQUIRE(gguf_types && weights && outputs && out_features, "matvec_group_norm received a null array");
    NormIn nrm;
    int st = check_norm("matvec_group_norm", x, norm, in_f, &nrm);
    if (st) return st;
    int kinds[3];
    long long rows = 0;
    int f16 = 0;
    for (int i = 0; i < count; ++i) {
        REQUIRE(fused_type_ok(gguf_types[i]), "matvec_group_norm: GGUF type %d is not Q4_K, Q6_K or F16",
                gguf_types[i]);
        st = check_matvec("matvec_group_norm", weights[i], x, outputs[i], in_f, out_features[i],
                          fused_walign(gguf_types[i]), 2);
        if (st) return st;
        kinds[i] = fused_kind(gguf_types[i]);
        f16 += kinds[i] == 1;
        rows += out_features[i];
    }
    REQUIRE(rows <= INT_MAX, "matvec_group_norm: %lld rows in total exceed INT_MAX", rows);
    if (f16 != 0 && f16 != count)
        return fail(CITLALI_ERR_UNSUPPORTED, "matvec_group_norm: F16 and quantized weights have no grouped kernel");
    if (!norm_length_ok(in_f))
        return fail(CITLALI_ERR_UNSUPPORTED, "matvec_group_norm: in_features %d has no grouped kernel", in_f);
    HIP_TRY(launch_matvec_group(count, kinds, weights, x, outputs, out_features, in_f, &nrm, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_matvec_gate_up_swiglu_norm(int gguf_type, const uint8_t* w_gate, const uint8_t* w_up,
                                                          const uint16_t* x, const citlali_hip_norm* norm,
                                                          uint16_t* act, int in_f, int out_f) {
    REQUIRE(fused_type_ok(gguf_type), "matvec_gate_up_swiglu_norm: GGUF type %d is not Q4_K, Q6_K or F16",
            gguf_type);
    NormIn nrm;
    int st = check_norm("matvec_gate_up_swiglu_norm", x, norm, in_f, &nrm);
    if (st) return st;
    const uintptr_t walign = fused_walign(gguf_type);
    st = check_matvec("matvec_gate_up_swiglu_norm", w_gate, x, act, in_f, out_f, walign, 2);
    if (st) return st;
    REQUIRE(w_up && aligned(w_up, walign), "matvec_gate_up_swiglu_norm: bad up weight");
    if (!gate_up_length_ok(in_f))
        return fail(CITLALI_ERR_UNSUPPORTED, "matvec_gate_up_swiglu_norm: in_features %d has no fused kernel", in_f);
    HIP_TRY(launch_matvec_gate_up_swiglu(fused_kind(gguf_type), w_gate, w_up, x, act, in_f, out_f, &nrm,
                                         g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_matvec_norm(int gguf_type, const uint8_t* w, const uint16_t* x,
                                           const citlali_hip_norm* norm, void* y, int f32_out, int in_f, int out_f) {
    REQUIRE(fused_type_ok(gguf_type), "matvec_norm: GGUF type %d is not Q4_K, Q6_K or F16", gguf_type);
    NormIn nrm;
    int st = check_norm("matvec_norm", x, norm, in_f, &nrm);
    if (st) return st;
    st = check_matvec("matvec_norm", w, x, y, in_f, out_f, fused_walign(gguf_type), f32_out ? 4 : 2);
    if (st) return st;
    if (!norm_length_ok(in_f))
        return fail(CITLALI_ERR_UNSUPPORTED, "matvec_norm: in_features %d has no prologue kernel", in_f);
    HIP_TRY(launch_matvec_norm(fused_kind(gguf_type), w, x, nrm, y, f32_out != 0, in_f, out_f, g_stream));
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_set_kernel_timing(void* start, void* stop) {
    REQUIRE((start == nullptr) == (stop == nullptr), "set_kernel_timing: give both events or neither");
    KernelTiming& t = kernel_timing();
    REQUIRE(start == nullptr || t.starts.empty(), "set_kernel_timing: per-dispatch timing is armed");
    t.start = static_cast<hipEvent_t>(start);
    t.stop = static_cast<hipEvent_t>(stop);
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_set_dispatch_timing(void* const* starts, void* const* stops, int n) {
    REQUIRE(n >= 0 && n <= CITLALI_MAX_TIMED_DISPATCHES, "set_dispatch_timing: n = %d outside [0, %d]", n,
            CITLALI_MAX_TIMED_DISPATCHES);
    KernelTiming& t = kernel_timing();
    if (n == 0) {   // disarm; the count stays readable
        t.starts.clear();
        t.stops.clear();
        return CITLALI_OK;
    }
    REQUIRE(starts != nullptr && stops != nullptr, "set_dispatch_timing: null event array");
    REQUIRE(t.start == nullptr, "set_dispatch_timing: call-span timing is armed");
    for (int i = 0; i < n; ++i)
        REQUIRE(starts[i] != nullptr && stops[i] != nullptr, "set_dispatch_timing: null event in pair %d", i);
    t.starts.assign(reinterpret_cast<const hipEvent_t*>(starts), reinterpret_cast<const hipEvent_t*>(starts) + n);
    t.stops.assign(reinterpret_cast<const hipEvent_t*>(stops), reinterpret_cast<const hipEvent_t*>(stops) + n);
    t.used = 0;
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_dispatch_timing_count(int* count) {
    REQUIRE(count, "null output pointer");
    *count = kernel_timing().used;
    return CITLALI_OK;
}

CITLALI_EXPORT int citlali_hip_event_create(void** ev) {
    REQUIRE(ev, "null output pointer");
    hipEvent_t e = nullptr;
    HIP_TRY(hipEventCreate(&e));
    *ev = e;
    return CITLALI_OK;
}
CITLALI_EXPORT int citlali_hip_event_record(void* ev) {
    REQUIRE(ev, "null event");
    HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(ev), g_stream));
    return CITLALI_OK;
}
CITLALI_EXPORT int citlali_hip_event_synchronize(void* ev) {
    REQUIRE(ev, "null event");
    HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(ev)));
    return CITLALI_OK;
}
CITLALI_EXPORT int citlali_hip_event_elapsed_ms(void* a, void* b, float* ms) {
    REQUIRE(a && b && ms, "null event");
    HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b)));
    return CITLALI_OK;
}
CITLALI_EXPORT int citlali_hip_event_destroy(void* ev) {
    if (ev) HIP_TRY(hipEventDestroy(static_cast<hipEvent_t>(ev)));
    return CITLALI_OK;
}
