// linear_backend.cpp -- Fp16LinearBackend: the weight-kind dispatch of the
// reference (src/model/linear_backend.cpp:9-68), same cases and messages,
// plus size checks of the three buffers so a mismatched handle throws
// instead of reading or writing past a buffer.
#include "citlali/model/linear_backend.h"

#include "citlali/common.h"
#include "citlali/compute/hip/kernels.h"

#include <limits>
#include <string>

namespace citlali::model {
namespace {

int as_int(uint64_t value, const std::string& label) {
    require(value <= static_cast<uint64_t>(std::numeric_limits<int>::max()),
            label + " is too large for this minimal kernel path");
    return static_cast<int>(value);
}

void require_bytes(const compute::DeviceBufferPtr& buf, uint64_t need, const std::string& what) {
    const uint64_t have = buf ? buf->bytes() : 0;
    require(have >= need, what + " holds " + std::to_string(have) + " bytes, " + std::to_string(need) +
                              " needed");
}

class Fp16LinearBackend final : public LinearBackend {
public:
    void forward(const WeightHandle& weight, const compute::DeviceBufferPtr& input,
                 const compute::DeviceBufferPtr& output) const override {
        require(input && output, "linear backend received a null buffer");
        const int in_f = as_int(weight.cols(), weight.name + " cols");
        const int out_f = as_int(weight.rows(), weight.name + " rows");
        switch (weight.storage_kind) {
            case compute::WeightStorageKind::QuantizedDevice: {
                if (weight.gguf_type != compute::GgufTensorType::Q4_K &&
                    weight.gguf_type != compute::GgufTensorType::Q6_K)
                    throw Error("unsupported weight storage kind for: " + weight.name);
                check_sizes(weight, input, output, in_f, out_f);
                if (weight.gguf_type == compute::GgufTensorType::Q4_K)
                    compute::launch_matvec_q4k(weight.device_quantized_data(), input->half_data(),
                                               output->half_data(), in_f, out_f);
                else
                    compute::launch_matvec_q6k(weight.device_quantized_data(), input->half_data(),
                                               output->half_data(), in_f, out_f);
                return;
            }
            case compute::WeightStorageKind::Fp16Device:
                check_sizes(weight, input, output, in_f, out_f);
                compute::launch_matvec_fp16(weight.device_half_data(), input->half_data(), output->half_data(),
                                            in_f, out_f);
                return;
        }
        throw Error("unknown storage_kind");
    }

private:
    static void check_sizes(const WeightHandle& w, const compute::DeviceBufferPtr& input,
                            const compute::DeviceBufferPtr& output, int in_f, int out_f) {
        const compute::GgufTensorType t = w.storage_kind == compute::WeightStorageKind::Fp16Device
                                              ? compute::GgufTensorType::F16
                                              : w.gguf_type;
        require_bytes(w.buffer, compute::gguf_tensor_nbytes(t, (uint64_t)in_f * (uint64_t)out_f),
                      w.name + " weight buffer");
        require_bytes(input, (uint64_t)in_f * 2, w.name + " input buffer");
        require_bytes(output, (uint64_t)out_f * 2, w.name + " output buffer");
    }
};

}  // namespace

std::unique_ptr<LinearBackend> make_fp16_linear_backend() { return std::make_unique<Fp16LinearBackend>(); }

}  // namespace citlali::model
