// citlali/model/linear_backend.h -- y = W x for one weight.
//
// Same interface as the reference (include/citlali/model/linear_backend.h:10-21):
// forward(weight, input, output) dispatches on the weight's storage kind and
// GGUF type to the gfx950 GEMVs (Q4_K, Q6_K fused dequant; fp16).
#pragma once

#include "citlali/compute/hip/tensor.h"
#include "citlali/model/weight_handle.h"

#include <memory>

namespace citlali::model {

class LinearBackend {
public:
    virtual ~LinearBackend() = default;
    virtual void forward(const WeightHandle& weight, const compute::DeviceBufferPtr& input,
                         const compute::DeviceBufferPtr& output) const = 0;
};

std::unique_ptr<LinearBackend> make_fp16_linear_backend();

}  // namespace citlali::model
