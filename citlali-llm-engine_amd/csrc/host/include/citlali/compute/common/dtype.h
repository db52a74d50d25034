// citlali/compute/common/dtype.h -- GGUF tensor type tags, block geometry and
// the host fp16 conversion rules.
//
// Interface of the reference's include/citlali/compute/common/dtype.h:14-106
// (names, enum values and results are the GGUF format and the reference's
// host rounding rule; the implementation is this library's own).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

namespace citlali::compute {

// GGUF `ggml_type` codes of the tensors the reference knows (dtype.h:14-31).
enum class GgufTensorType : uint32_t {
    F32 = 0,
    F16 = 1,
    Q4_0 = 2,
    Q4_1 = 3,
    Q5_0 = 6,
    Q5_1 = 7,
    Q8_0 = 8,
    Q8_1 = 9,
    Q2_K = 10,
    Q3_K = 11,
    Q4_K = 12,
    Q5_K = 13,
    Q6_K = 14,
    Q8_K = 15,
    BF16 = 30,
    Unknown = 0xffffffffu,
};

// How a weight lives on the device (dtype.h:33-39): fp16 values, or the raw
// quantised super-blocks consumed by the fused-dequant GEMVs.
enum class WeightStorageKind {
    Fp16Device,
    QuantizedDevice,
};

std::string to_string(GgufTensorType type);   // "Q4_K", ...; "Unknown" otherwise
// Elements per block and bytes per block; 0 for types the engine cannot
// store (dtype.cpp:28-57: F32, F16, BF16, Q8_0, Q4_K, Q6_K are known).
std::size_t gguf_type_block_size(GgufTensorType type);
std::size_t gguf_type_block_bytes(GgufTensorType type);
// ceil(elements / block) * block_bytes; 0 for an unknown type.
std::size_t gguf_tensor_nbytes(GgufTensorType type, std::size_t elements);

// Host fp16 rules of the reference (dtype.cpp:67-176): float -> fp16 rounds
// to nearest with ties away from zero, sends overflow and NaN to +-Inf and
// magnitudes below 2^-25 to +-0; fp16 -> float is exact; bf16 -> fp16 goes
// through float.
uint16_t float_to_half_bits(float value);
float half_bits_to_float(uint16_t bits);
uint16_t bfloat16_to_half_bits(uint16_t value);

}  // namespace citlali::compute
