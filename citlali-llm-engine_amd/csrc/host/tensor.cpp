// tensor.cpp -- DeviceBuffer over the C ABI (reference: tensor.cu:9-104).
#include "citlali/compute/hip/tensor.h"

#include "citlali/common.h"
#include "citlali/compute/hip/hip_check.h"

#include <string>

namespace citlali::compute {

DeviceBuffer::DeviceBuffer(std::size_t bytes) { allocate(bytes); }

DeviceBuffer::~DeviceBuffer() { reset(); }

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept : data_(other.data_), bytes_(other.bytes_) {
    other.data_ = nullptr;
    other.bytes_ = 0;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
    if (this != &other) {
        reset();
        data_ = other.data_;
        bytes_ = other.bytes_;
        other.data_ = nullptr;
        other.bytes_ = 0;
    }
    return *this;
}

void DeviceBuffer::allocate(std::size_t bytes) {
    reset();
    if (bytes == 0) return;
    void* p = nullptr;
    CITLALI_HIP_CHECK(citlali_hip_malloc(&p, bytes));
    data_ = p;
    bytes_ = bytes;
}

void DeviceBuffer::reset() {
    if (!data_) return;
    (void)citlali_hip_free(data_);   // like the reference, a failed free is not reported
    data_ = nullptr;
    bytes_ = 0;
}

void DeviceBuffer::copy_from_host(const void* source, std::size_t bytes) {
    require(bytes <= bytes_, "copy_from_host: " + std::to_string(bytes) + " bytes into a buffer of " +
                                 std::to_string(bytes_));
    CITLALI_HIP_CHECK(citlali_hip_memcpy_h2d(data_, source, bytes));
}

void DeviceBuffer::copy_to_host(void* target, std::size_t bytes) const {
    require(bytes <= bytes_, "copy_to_host: " + std::to_string(bytes) + " bytes from a buffer of " +
                                 std::to_string(bytes_));
    CITLALI_HIP_CHECK(citlali_hip_memcpy_d2h(target, data_, bytes));
}

DeviceBufferPtr make_device_buffer(std::size_t bytes) { return std::make_shared<DeviceBuffer>(bytes); }

DeviceBufferPtr make_device_half_buffer(std::size_t elements) {
    return make_device_buffer(elements * sizeof(uint16_t));
}

}  // namespace citlali::compute
