#pragma once
#include <string>
#include <ostream>
#include <vector>
#include <memory>
#include "core/device.h"
#include "core/dtype.h"

namespace ormi {
    // Owns one device allocation and hands it back to its device's allocator
    // pool on destruction (reference: csrc/core/memory.h:9-20, memory.cpp:12-17).
    // dtype is additive; every reference call site keeps Float32.
    struct Buffer {
        void* ptr;
        size_t bytes;
        std::vector<int> shape;
        Device device;
        DType dtype;

        Buffer(void* p, size_t b, std::vector<int> s, Device d, DType dt = DType::Float32);
        ~Buffer();
        Buffer(const Buffer&) = delete;
        Buffer& operator=(const Buffer&) = delete;

        size_t numel() const { return bytes / dtype_size(dtype); }
    };

    std::string to_string(const Buffer& buffer);
    std::string to_string(const std::shared_ptr<Buffer>& buffer);
    std::ostream& operator<<(std::ostream& os, const Buffer& buffer);

    std::shared_ptr<Buffer> empty(std::vector<int> shape, DeviceEnum dev, DType dtype = DType::Float32);
    std::shared_ptr<Buffer> full(std::vector<int> shape, float fill_value, DeviceEnum dev);
    std::shared_ptr<Buffer> scalar(float val, DeviceEnum dev);
    std::shared_ptr<Buffer> zeros(std::vector<int> shape, DeviceEnum dev);
    std::shared_ptr<Buffer> ones(std::vector<int> shape, DeviceEnum dev);
    std::shared_ptr<Buffer> zeros_like(std::shared_ptr<Buffer> array);
    std::shared_ptr<Buffer> zeros_like(std::shared_ptr<Buffer> array, DeviceEnum dev);
    std::shared_ptr<Buffer> ones_like(std::shared_ptr<Buffer> array);
    std::shared_ptr<Buffer> ones_like(std::shared_ptr<Buffer> array, DeviceEnum dev);
}
