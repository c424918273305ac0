#pragma once
// Device descriptor of the dl:: API (include/dl/core/Device.hpp in the
// reference).  DeviceType::CUDA keeps its public name for source
// compatibility; in this build it denotes the HIP device (an MI355X).

#include <string>

namespace dl {

enum class DeviceType {
    CPU,
    CUDA
};

class Device {
public:
    DeviceType type;
    int index;

    Device(DeviceType type = DeviceType::CUDA, int index = 0);

    bool is_cuda() const;
    bool is_cpu() const;
    std::string str() const;
};

}  // namespace dl

using DeviceType = dl::DeviceType;
using Device = dl::Device;
