// citlali/compute/hip/tensor.h -- owning device buffer.
//
// Same interface as the reference's DeviceBuffer (tensor.h:10-54): move-only,
// `allocate` frees then allocates, `reset` frees and ignores the free status,
// copies are blocking.  Unlike the reference, a copy larger than the buffer
// throws instead of writing past it.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>

namespace citlali::compute {

class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(std::size_t bytes);
    ~DeviceBuffer();

    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& other) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept;

    void allocate(std::size_t bytes);   // bytes == 0 leaves the buffer empty
    void reset();

    void copy_from_host(const void* source, std::size_t bytes);
    void copy_to_host(void* target, std::size_t bytes) const;   // waits for queued work

    void* data() { return data_; }
    const void* data() const { return data_; }
    std::size_t bytes() const { return bytes_; }
    uint16_t* half_data() { return static_cast<uint16_t*>(data_); }
    const uint16_t* half_data() const { return static_cast<const uint16_t*>(data_); }

private:
    void* data_ = nullptr;
    std::size_t bytes_ = 0;
};

using DeviceBufferPtr = std::shared_ptr<DeviceBuffer>;
DeviceBufferPtr make_device_buffer(std::size_t bytes);
DeviceBufferPtr make_device_half_buffer(std::size_t elements);

}  // namespace citlali::compute
