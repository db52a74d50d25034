// citlali/model/weight_loader.h -- GGUF tensors into device memory.
//
// Same class and policies as the reference's WeightLoader
// (include/citlali/model/weight_loader.h:14-61, src/model/weight_loader.cpp:
// 337-467).  KeepQuantized keeps the raw GGUF blocks of a quantised type
// (storage QuantizedDevice, the fused-dequant GEMVs read them); everything
// else becomes fp16 (storage Fp16Device): F16 as is, F32 / BF16 / Q8_0
// through the host fp16 rule, Q4_K / Q6_K on the device with the kernels
// that reproduce the host routines bit for bit.  Tensor bytes go from the
// GGUF file's mapping straight to the device.
#pragma once

#include "citlali/io/gguf_reader.h"
#include "citlali/model/weight_handle.h"

#include <string>

namespace citlali::model {

// The GGUF block-quantised types the reference keeps as raw blocks under
// KeepQuantized (weight_loader.cpp:343-374).
bool is_quantized_type(compute::GgufTensorType type);

class WeightLoader {
public:
    explicit WeightLoader(const io::GgufFile& gguf, WeightLoadPolicy policy = WeightLoadPolicy::DequantizeToFp16);

    // Throws citlali::Error "missing required tensor: <name>" when absent,
    // or when the type has no fp16 conversion.
    WeightHandle load_required(const std::string& name) const;
    // Name, type and dims only, no device buffer (the reference fills these
    // for layers run elsewhere, weight_loader.cpp:412-421).
    WeightHandle load_remote_required(const std::string& name) const;
    // An empty handle when the tensor is absent.
    WeightHandle load_optional(const std::string& name) const;

    WeightLoadPolicy policy() const { return policy_; }

private:
    const io::GgufFile& gguf_;
    WeightLoadPolicy policy_;
};

}  // namespace citlali::model
