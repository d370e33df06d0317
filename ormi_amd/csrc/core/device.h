#pragma once
#include <string>
#include <stdexcept>

namespace ormi {
    // CPU=0 and CUDA=1 keep the reference numbering (csrc/core/device.h:6);
    // HIP is the MI355X device this library provides.
    enum class DeviceEnum { CPU = 0, CUDA = 1, HIP = 2 };

    struct Device {
        DeviceEnum type;
        int id;

        // The reference defaults the C++ Device to CUDA (csrc/core/device.h:12);
        // the default is kept so Device() means the same thing in both.
        Device(DeviceEnum t = DeviceEnum::CUDA, int i = 0) : type(t), id(i) {}

        std::string to_string() const {
            std::string t;
            switch (type) {
                case DeviceEnum::CPU:  t = "cpu"; break;
                case DeviceEnum::CUDA: t = "cuda"; break;
                case DeviceEnum::HIP:  t = "hip"; break;
                default: throw std::runtime_error("ormi::Device - Unknown DeviceEnum");
            }
            return t + ":" + std::to_string(id);
        }

        bool operator==(const Device& o) const { return type == o.type && id == o.id; }
        bool operator!=(const Device& o) const { return !(*this == o); }
    };
}
