// weight_loader.cpp -- WeightLoader (policies of weight_loader.cpp:337-467 of
// the reference).
//
// Conversions to fp16 under DequantizeToFp16, as the reference's
// load_as_fp16 (weight_loader.cpp:71-139, 451-467):
//   F16   the bits as stored
//   F32   float_to_half_bits(value)
//   BF16  bfloat16_to_half_bits(value)
//   Q8_0  blocks of 34 bytes (fp16 d, 32 int8 q): float_to_half_bits(d * q)
//   Q4_K, Q6_K  the host dequant rule, run on the device
// F32 / BF16 / Q8_0 are converted on the host (norm vectors in the Qwen
// files); the K-quants, which hold nearly all of a model's bytes, are copied
// as blocks and expanded in device memory.
#include "citlali/model/weight_loader.h"

#include "citlali/common.h"
#include "citlali/compute/hip/kernels.h"

#include <sys/mman.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <vector>

namespace citlali::model {

using compute::GgufTensorType;

namespace {
// Maps the file pages of a tensor's bytes in one call before they are copied
// (MADV_POPULATE_READ, Linux 5.14 and later): one pass over the range in the
// kernel instead of a page fault per 4 KB page inside the copy.  Where the
// kernel does not know the advice the copy faults the pages in as before.
void prefault(const uint8_t* p, uint64_t n) {
    static const uintptr_t page = static_cast<uintptr_t>(sysconf(_SC_PAGESIZE));
    const uintptr_t a = reinterpret_cast<uintptr_t>(p) & ~(page - 1);
    const uintptr_t e = reinterpret_cast<uintptr_t>(p) + n;
    (void)::madvise(reinterpret_cast<void*>(a), e - a, MADV_POPULATE_READ);
}
}  // namespace

bool is_quantized_type(GgufTensorType t) {
    switch (t) {
        case GgufTensorType::Q2_K:
        case GgufTensorType::Q3_K:
        case GgufTensorType::Q4_0:
        case GgufTensorType::Q4_1:
        case GgufTensorType::Q4_K:
        case GgufTensorType::Q5_0:
        case GgufTensorType::Q5_1:
        case GgufTensorType::Q5_K:
        case GgufTensorType::Q6_K:
        case GgufTensorType::Q8_0:
        case GgufTensorType::Q8_1:
        case GgufTensorType::Q8_K: return true;
        default: return false;
    }
}

namespace {

template <typename Convert>
std::vector<uint16_t> convert_host(uint64_t count, Convert f) {
    std::vector<uint16_t> out(static_cast<size_t>(count));
    for (uint64_t i = 0; i < count; ++i) out[static_cast<size_t>(i)] = f(i);
    return out;
}

std::vector<uint16_t> q8_0_to_half(const uint8_t* src, uint64_t count) {
    constexpr uint64_t kBlock = 32, kBytes = 2 + kBlock;
    return convert_host(count, [&](uint64_t i) {
        const uint8_t* b = src + (i / kBlock) * kBytes;
        uint16_t dh;
        std::memcpy(&dh, b, 2);
        const float d = compute::half_bits_to_float(dh);
        const int8_t q = static_cast<int8_t>(b[2 + i % kBlock]);
        return compute::float_to_half_bits(d * static_cast<float>(q));
    });
}

}  // namespace

WeightLoader::WeightLoader(const io::GgufFile& gguf, WeightLoadPolicy policy) : gguf_(gguf), policy_(policy) {}

WeightHandle WeightLoader::load_required(const std::string& name) const {
    const io::GgufTensorInfo* t = gguf_.find_tensor(name);
    require(t != nullptr, "missing required tensor: " + name);

    WeightHandle h;
    h.name = name;
    h.gguf_type = t->type;
    h.storage_kind = compute::WeightStorageKind::Fp16Device;
    h.dims = t->dims;
    h.element_count = t->element_count();
    const uint8_t* src = gguf_.tensor_data(*t);
    const uint64_t n = h.element_count;
    if (t->nbytes >= (uint64_t(1) << 20)) prefault(src, t->nbytes);

    if (policy_ == WeightLoadPolicy::KeepQuantized && is_quantized_type(t->type)) {
        h.storage_kind = compute::WeightStorageKind::QuantizedDevice;
        h.buffer = compute::make_device_buffer(static_cast<size_t>(t->nbytes));
        h.buffer->copy_from_host(src, static_cast<size_t>(t->nbytes));
        return h;
    }

    std::vector<uint16_t> host;
    switch (t->type) {
        case GgufTensorType::F16:
            h.buffer = compute::make_device_half_buffer(static_cast<size_t>(n));
            h.buffer->copy_from_host(src, static_cast<size_t>(n) * 2);
            return h;
        case GgufTensorType::Q4_K:
        case GgufTensorType::Q6_K: {
            h.buffer = compute::make_device_half_buffer(static_cast<size_t>(n));
            compute::DeviceBuffer blocks(static_cast<size_t>(t->nbytes));
            blocks.copy_from_host(src, static_cast<size_t>(t->nbytes));
            const auto* b = static_cast<const uint8_t*>(blocks.data());
            if (t->type == GgufTensorType::Q4_K) {
                compute::launch_dequant_q4k_f16(b, n, h.buffer->half_data());
            } else {
                compute::launch_dequant_q6k_f16(b, n, h.buffer->half_data());
            }
            compute::synchronize();   // before the block buffer is freed
            return h;
        }
        case GgufTensorType::F32:
            host = convert_host(n, [&](uint64_t i) {
                float v;
                std::memcpy(&v, src + 4 * i, 4);
                return compute::float_to_half_bits(v);
            });
            break;
        case GgufTensorType::BF16:
            host = convert_host(n, [&](uint64_t i) {
                uint16_t v;
                std::memcpy(&v, src + 2 * i, 2);
                return compute::bfloat16_to_half_bits(v);
            });
            break;
        case GgufTensorType::Q8_0: host = q8_0_to_half(src, n); break;
        default:
            throw Error("tensor type is not implemented by the FP16 loader yet: " + name +
                        " type=" + compute::to_string(t->type));
    }
    h.buffer = compute::make_device_half_buffer(static_cast<size_t>(n));
    h.buffer->copy_from_host(host.data(), host.size() * sizeof(uint16_t));
    return h;
}

WeightHandle WeightLoader::load_remote_required(const std::string& name) const {
    const io::GgufTensorInfo* t = gguf_.find_tensor(name);
    require(t != nullptr, "missing required tensor: " + name);
    WeightHandle h;
    h.name = name;
    h.gguf_type = t->type;
    h.dims = t->dims;
    h.element_count = t->element_count();
    return h;
}

WeightHandle WeightLoader::load_optional(const std::string& name) const {
    if (gguf_.find_tensor(name) == nullptr) return {};
    return load_required(name);
}

}  // namespace citlali::model
