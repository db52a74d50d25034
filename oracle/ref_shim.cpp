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
