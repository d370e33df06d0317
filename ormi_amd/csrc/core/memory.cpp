#include <stdexcept>
#include <sstream>
#include <iomanip>
#include <cmath>
#include <cstring>
#include "core/memory.h"
#include "core/allocator.h"

namespace ormi {
    Buffer::Buffer(void* p, size_t b, std::vector<int> s, Device d, DType dt)
        : ptr(p), bytes(b), shape(std::move(s)), device(d), dtype(dt) {}

    Buffer::~Buffer() {
        if (ptr) get_allocator(device.type)->free(ptr, bytes);
    }

    static double element_as_double(const unsigned char* base, size_t i, DType dt) {
        switch (dt) {
            case DType::Float32: { float v; std::memcpy(&v, base + 4 * i, 4); return v; }
            case DType::Int32:   { int32_t v; std::memcpy(&v, base + 4 * i, 4); return v; }
            case DType::Bool:    return base[i] ? 1.0 : 0.0;
            case DType::Int64:   { int64_t v; std::memcpy(&v, base + 8 * i, 8); return (double)v; }
            case DType::BFloat16: {
                uint16_t h; std::memcpy(&h, base + 2 * i, 2);
                uint32_t u = (uint32_t)h << 16; float f; std::memcpy(&f, &u, 4); return f;
            }
            case DType::Float16: {
                uint16_t h; std::memcpy(&h, base + 2 * i, 2);
                const int sign = h >> 15, exp = (h >> 10) & 31, man = h & 1023;
                double v = exp == 0 ? man * 0x1p-24 : exp == 31 ? (man ? NAN : INFINITY)
                                                                : (1.0 + man / 1024.0) * std::ldexp(1.0, exp - 15);
                return sign ? -v : v;
            }
        }
        return 0.0;
    }

    static void format_tensor(std::ostringstream& oss, const unsigned char* data, DType dt,
                              const std::vector<int>& shape, const std::vector<size_t>& strides,
                              size_t dim, size_t offset) {
        if (shape.empty()) { oss << element_as_double(data, offset, dt); return; }
        oss << "[";
        for (int i = 0; i < shape[dim]; ++i) {
            const size_t off = offset + (size_t)i * strides[dim];
            if (dim == shape.size() - 1) oss << element_as_double(data, off, dt);
            else format_tensor(oss, data, dt, shape, strides, dim + 1, off);
            if (i < shape[dim] - 1) {
                if (dim == shape.size() - 1) oss << ", ";
                else oss << ",\n" << std::string(dim + 1, ' ');
            }
        }
        oss << "]";
    }

    // Pretty-printer in the reference's format (csrc/core/memory.cpp:19-71).
    std::string to_string(const Buffer& buffer) {
        std::vector<size_t> strides(buffer.shape.size(), 1);
        for (int i = (int)buffer.shape.size() - 2; i >= 0; --i) strides[i] = strides[i + 1] * buffer.shape[i + 1];
        std::vector<unsigned char> host(buffer.bytes);
        get_allocator(buffer.device.type)->copy_device_to_host(host.data(), buffer.ptr, buffer.bytes);
        std::ostringstream oss;
        oss << std::fixed << std::setprecision(4);
        format_tensor(oss, host.data(), buffer.dtype, buffer.shape, strides, 0, 0);
        return oss.str();
    }

    std::string to_string(const std::shared_ptr<Buffer>& buffer) {
        return buffer ? to_string(*buffer) : std::string("null");
    }

    std::ostream& operator<<(std::ostream& os, const Buffer& buffer) { return os << to_string(buffer); }

    std::shared_ptr<Buffer> empty(std::vector<int> shape, DeviceEnum dev, DType dtype) {
        size_t bytes = dtype_size(dtype);
        for (int d : shape) {
            if (d < 0) throw std::runtime_error("Negative dimension in shape.");
            bytes *= (size_t)d;
        }
        IAllocator* alloc = get_allocator(dev);
        void* ptr = bytes ? alloc->allocate(bytes) : nullptr;
        return std::make_shared<Buffer>(ptr, bytes, std::move(shape), Device(dev), dtype);
    }

    std::shared_ptr<Buffer> full(std::vector<int> shape, float fill_value, DeviceEnum dev) {
        auto buf = empty(shape, dev);
        const size_t n = buf->numel();
        if (n) get_allocator(dev)->fill_n(buf->ptr, &fill_value, n, DType::Float32);
        return buf;
    }

    std::shared_ptr<Buffer> scalar(float v, DeviceEnum dev) { return full({1}, v, dev); }
    std::shared_ptr<Buffer> zeros(std::vector<int> s, DeviceEnum dev) { return full(std::move(s), 0.0f, dev); }
    std::shared_ptr<Buffer> ones(std::vector<int> s, DeviceEnum dev) { return full(std::move(s), 1.0f, dev); }
    std::shared_ptr<Buffer> zeros_like(std::shared_ptr<Buffer> a) { return full(a->shape, 0.0f, a->device.type); }
    std::shared_ptr<Buffer> zeros_like(std::shared_ptr<Buffer> a, DeviceEnum dev) { return full(a->shape, 0.0f, dev); }
    std::shared_ptr<Buffer> ones_like(std::shared_ptr<Buffer> a) { return full(a->shape, 1.0f, a->device.type); }
    std::shared_ptr<Buffer> ones_like(std::shared_ptr<Buffer> a, DeviceEnum dev) { return full(a->shape, 1.0f, dev); }
}
