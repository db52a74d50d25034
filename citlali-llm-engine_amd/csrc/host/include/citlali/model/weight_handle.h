// citlali/model/weight_handle.h -- a loaded weight tensor.
//
// Same fields and accessors as the reference's WeightHandle
// (include/citlali/model/weight_loader.h:20-42).  dims = [cols, rows] in GGUF
// order: cols() = dims[0] = in_features, rows() = dims[1] = out_features
// (linear_backend.cpp:35-36 passes them as (in, out)).
#pragma once

#include "citlali/compute/common/dtype.h"
#include "citlali/compute/hip/tensor.h"

#include <cstdint>
#include <string>
#include <vector>

namespace citlali::model {

enum class WeightLoadPolicy {
    DequantizeToFp16,
    KeepQuantized,
};

struct WeightHandle {
    std::string name;
    compute::GgufTensorType gguf_type = compute::GgufTensorType::Unknown;
    compute::WeightStorageKind storage_kind = compute::WeightStorageKind::Fp16Device;
    std::vector<uint64_t> dims;
    compute::DeviceBufferPtr buffer;
    uint64_t element_count = 0;

    uint64_t cols() const { return dims.empty() ? 0 : dims[0]; }
    uint64_t rows() const { return dims.size() < 2 ? 1 : dims[1]; }

    const uint16_t* device_half_data() const { return buffer ? buffer->half_data() : nullptr; }
    uint16_t* device_half_data() { return buffer ? buffer->half_data() : nullptr; }
    const uint8_t* device_quantized_data() const {
        return buffer ? static_cast<const uint8_t*>(buffer->data()) : nullptr;
    }
    uint8_t* device_quantized_data() { return buffer ? static_cast<uint8_t*>(buffer->data()) : nullptr; }
};

}  // namespace citlali::model
