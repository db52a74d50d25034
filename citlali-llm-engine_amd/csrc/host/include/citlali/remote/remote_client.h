// citlali/remote/remote_client.h -- the option types of the reference's
// remote layer offload (include/citlali/remote/remote_client.h:12-25), so
// that callers written against QwenModel::load / InferenceSession::load_model
// with a RemoteOptions argument compile unchanged.
//
// The offload itself (RemoteClient: the USB / Wi-Fi transport to a second
// device, src/remote/remote_client.cpp) is not part of this build.  A load
// whose options name layers to offload is refused with citlali::Error after
// the reference's own range check; options with no layers load every layer
// on the GPU, as the reference does when nothing is offloaded.
#pragma once

#include <algorithm>
#include <cstdint>
#include <string>
#include <vector>

namespace citlali::remote {

enum class Backend { Auto, Gpu, Npu, Hybrid };
enum class Transport { Usb, Wifi6 };

struct RemoteOptions {
    std::string endpoint;
    Transport transport = Transport::Usb;
    Backend backend = Backend::Gpu;
    std::vector<std::uint32_t> layers;

    // an endpoint and at least one layer (remote_client.h:21-23)
    bool enabled() const { return !endpoint.empty() && !layers.empty(); }
    // listed in `layers` (remote_client.cpp:364-366)
    bool offloads_layer(std::uint32_t layer_index) const {
        return std::find(layers.begin(), layers.end(), layer_index) != layers.end();
    }
};

}  // namespace citlali::remote
