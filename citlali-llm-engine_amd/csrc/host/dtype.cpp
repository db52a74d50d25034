// dtype.cpp -- GGUF type table and the host fp16 rules (dtype.cpp:7-176 of
// the reference restated from the GGUF format and the rounding rule).
#include "citlali/compute/common/dtype.h"

#include <cstring>

namespace citlali::compute {
namespace {

struct TypeInfo {
    GgufTensorType type;
    const char* name;
    std::size_t block;   // elements per block, 0 if the engine cannot store it
    std::size_t bytes;   // bytes per block
};

// Q4_K: fp16 d, fp16 dmin, 12 B of 6-bit scales/mins, 128 B of nibbles.
// Q6_K: 128 B low nibbles, 64 B high bit pairs, 16 int8 scales, fp16 d.
// Q8_0: fp16 d + 32 int8.
constexpr TypeInfo kTypes[] = {
    {GgufTensorType::F32, "F32", 1, 4},        {GgufTensorType::F16, "F16", 1, 2},
    {GgufTensorType::Q4_0, "Q4_0", 0, 0},      {GgufTensorType::Q4_1, "Q4_1", 0, 0},
    {GgufTensorType::Q5_0, "Q5_0", 0, 0},      {GgufTensorType::Q5_1, "Q5_1", 0, 0},
    {GgufTensorType::Q8_0, "Q8_0", 32, 34},    {GgufTensorType::Q8_1, "Q8_1", 0, 0},
    {GgufTensorType::Q2_K, "Q2_K", 0, 0},      {GgufTensorType::Q3_K, "Q3_K", 0, 0},
    {GgufTensorType::Q4_K, "Q4_K", 256, 144},  {GgufTensorType::Q5_K, "Q5_K", 0, 0},
    {GgufTensorType::Q6_K, "Q6_K", 256, 210},  {GgufTensorType::Q8_K, "Q8_K", 0, 0},
    {GgufTensorType::BF16, "BF16", 1, 2},
};

const TypeInfo* find(GgufTensorType t) {
    for (const TypeInfo& i : kTypes)
        if (i.type == t) return &i;
    return nullptr;
}

uint32_t bits_of(float v) {
    uint32_t u;
    std::memcpy(&u, &v, sizeof u);
    return u;
}

float float_of(uint32_t u) {
    float v;
    std::memcpy(&v, &u, sizeof v);
    return v;
}

}  // namespace

std::string to_string(GgufTensorType type) {
    const TypeInfo* i = find(type);
    return i ? i->name : "Unknown";
}

std::size_t gguf_type_block_size(GgufTensorType type) {
    const TypeInfo* i = find(type);
    return i ? i->block : 0;
}

std::size_t gguf_type_block_bytes(GgufTensorType type) {
    const TypeInfo* i = find(type);
    return (i && i->block) ? i->bytes : 0;
}

std::size_t gguf_tensor_nbytes(GgufTensorType type, std::size_t elements) {
    const std::size_t block = gguf_type_block_size(type), bytes = gguf_type_block_bytes(type);
    if (block == 0 || bytes == 0) return 0;
    return (elements / block + (elements % block != 0)) * bytes;
}

// Nearest with ties away from zero: keep the fp16 significand, add the first
// dropped bit.  A carry out of the significand moves into the exponent, which
// is how 65520 becomes Inf.
uint16_t float_to_half_bits(float value) {
    const uint32_t u = bits_of(value);
    const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000u);
    const uint32_t mag = u & 0x7fffffffu;
    const int exp16 = static_cast<int>(mag >> 23) - (127 - 15);
    if (exp16 >= 31) return sign | 0x7c00u;                  // overflow, Inf and NaN
    if (exp16 >= 1) {
        const uint32_t h = (static_cast<uint32_t>(exp16) << 10) | ((mag >> 13) & 0x3ffu);
        return static_cast<uint16_t>(sign | (h + ((mag >> 12) & 1u)));
    }
    if (exp16 < -10) return sign;                            // below 2^-25
    // fp16 subnormal: the full significand shifted so its unit is 2^-24
    const uint32_t significand = (mag & 0x7fffffu) | 0x800000u;
    const int shift = 14 - exp16;                            // 14 .. 24
    const uint32_t h = (significand >> shift) + ((significand >> (shift - 1)) & 1u);
    return static_cast<uint16_t>(sign | h);
}

float half_bits_to_float(uint16_t bits) {
    const uint32_t sign = static_cast<uint32_t>(bits & 0x8000u) << 16;
    const uint32_t exp = (bits >> 10) & 0x1fu, man = bits & 0x3ffu;
    if (exp == 0x1f) return float_of(sign | 0x7f800000u | (man << 13));   // Inf, NaN payload kept
    if (exp != 0) return float_of(sign | ((exp + (127 - 15)) << 23) | (man << 13));
    if (man == 0) return float_of(sign);
    // subnormal man * 2^-24: normalise on its leading bit p (0..9)
    const int p = 31 - __builtin_clz(man);
    return float_of(sign | (static_cast<uint32_t>(p + 127 - 24) << 23) | ((man << (23 - p)) & 0x7fffffu));
}

uint16_t bfloat16_to_half_bits(uint16_t value) {
    return float_to_half_bits(float_of(static_cast<uint32_t>(value) << 16));
}

}  // namespace citlali::compute
