// ref_shim.cpp -- exposes the reference's own host fp16 and dequant routines
// through a C ABI so the tests can check the oracle restatement against them.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile into oracle/_ref/ from
// the reference sources where they lie (REF_ROOT, default /root/reference);
// nothing from the reference is copied into this repository.  The dequant
// routines live in an anonymous namespace of src/model/weight_loader.cpp, so
// this translation unit includes that file textually; the linker's section
// garbage collection drops the loader members that would need the CUDA
// DeviceBuffer, so no stand-in for any missing library is involved.
#include "src/model/weight_loader.cpp"

#include "citlali/compute/common/dtype.h"

#include <cstring>
#include <vector>

#define REF_API extern "C" __attribute__((visibility("default")))

// dtype.cpp:136-176
REF_API void ref_f2h_array(const float* in, uint64_t n, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = citlali::compute::float_to_half_bits(in[i]);
}

// dtype.cpp:76-133
REF_API void ref_h2f_array(const uint16_t* in, uint64_t n, float* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = citlali::compute::half_bits_to_float(in[i]);
}

// dtype.cpp:67-73
REF_API void ref_bf16_to_half_array(const uint16_t* in, uint64_t n, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = citlali::compute::bfloat16_to_half_bits(in[i]);
}

// weight_loader.cpp:147-237
REF_API void ref_dequant_q4k(const uint8_t* bytes, uint64_t nbytes, uint64_t count, uint16_t* out) {
    const std::vector<uint8_t> b(bytes, bytes + nbytes);
    const std::vector<uint16_t> v = citlali::model::dequant_q4_k(b, count);
    std::memcpy(out, v.data(), v.size() * sizeof(uint16_t));
}

// weight_loader.cpp:240-323
REF_API void ref_dequant_q6k(const uint8_t* bytes, uint64_t nbytes, uint64_t count, uint16_t* out) {
    const std::vector<uint8_t> b(bytes, bytes + nbytes);
    const std::vector<uint16_t> v = citlali::model::dequant_q6_k(b, count);
    std::memcpy(out, v.data(), v.size() * sizeof(uint16_t));
}

// dtype.cpp:28-64
REF_API uint64_t ref_tensor_nbytes(uint32_t type, uint64_t elements) {
    return citlali::compute::gguf_tensor_nbytes(static_cast<citlali::compute::GgufTensorType>(type), elements);
}

// ---- CPU baseline (bench.py's cpu_baseline leg) --------------------------
// The reference's CPU path for the hot path: its own load-time dequant
// (weight_loader.cpp:147-323, called through its std::vector API as the
// reference calls it) of each weight row to fp16 bits, widened with its
// half_bits_to_float (dtype.cpp:76-133), then an fp32 dot.  The reference
// has no CPU GEMV of its own, so the dot is this shim's; rows are split
// statically over `nthreads` OpenMP threads.
//
// variant (i): dequant + dot per call, the CPU analogue of the fused kernel.
REF_API void ref_matvec_dequant_dot(int type, const uint8_t* w, const uint16_t* x, float* y, int in_f, int out_f,
                                    int nthreads) {
    const size_t row_bytes = (size_t)in_f / 256 * (type == 12 ? 144 : 210);
    std::vector<float> xf(in_f);
    for (int k = 0; k < in_f; ++k) xf[k] = citlali::compute::half_bits_to_float(x[k]);
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int r = 0; r < out_f; ++r) {
        const std::vector<uint8_t> b(w + r * row_bytes, w + (r + 1) * row_bytes);
        const std::vector<uint16_t> v =
            type == 12 ? citlali::model::dequant_q4_k(b, (uint64_t)in_f) : citlali::model::dequant_q6_k(b, (uint64_t)in_f);
        float acc = 0.0f;
        for (int k = 0; k < in_f; ++k) acc += citlali::compute::half_bits_to_float(v[k]) * xf[k];
        y[r] = acc;
    }
}

// variant (ii): the fp32 dot over weights dequantised once beforehand (the
// reference's DequantizeToFp16 load policy), fp16 rows [out_f][in_f].
REF_API void ref_matvec_f16_dot(const uint16_t* wf16, const uint16_t* x, float* y, int in_f, int out_f, int nthreads) {
    std::vector<float> xf(in_f);
    for (int k = 0; k < in_f; ++k) xf[k] = citlali::compute::half_bits_to_float(x[k]);
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int r = 0; r < out_f; ++r) {
        const uint16_t* row = wf16 + (size_t)r * in_f;
        float acc = 0.0f;
        for (int k = 0; k < in_f; ++k) acc += citlali::compute::half_bits_to_float(row[k]) * xf[k];
        y[r] = acc;
    }
}
