#pragma once
#include <cstddef>
#include "core/device.h"
#include "core/dtype.h"

namespace ormi {
    // Device memory interface, same members and meaning as the reference's
    // (csrc/core/allocator.h:7-21). fill_n's third argument is an element
    // count, as in every reference implementation (cpu/allocator.cpp:49-53).
    class IAllocator {
    public:
        virtual ~IAllocator() = default;
        virtual void* allocate(size_t bytes) = 0;
        virtual void free(void* ptr, size_t bytes) = 0;
        virtual void memset(void* ptr, int value, size_t bytes) = 0;
        virtual void memcpy(void* dst, const void* src, size_t size) = 0;
        virtual void fill_n(void* dst, const void* val_ptr, size_t elements, DType dtype) = 0;
        virtual void copy_device_to_host(void* dst, const void* src, size_t bytes) = 0;
        virtual void copy_host_to_device(void* dst, const void* src, size_t bytes) = 0;
        virtual bool is_host_visible() const = 0;
    };

    using AllocatorGetter = IAllocator* (*)();

    // Devices plug their allocator in here; the reference hard-codes a switch
    // (csrc/core/allocator.cpp:5-12). The HIP allocator registers itself from
    // libormi_core; a CPU allocator is registered only by whoever loads one.
    void register_allocator(DeviceEnum dev, AllocatorGetter getter);
    bool has_allocator(DeviceEnum dev);
    IAllocator* get_allocator(DeviceEnum type);
    IAllocator* get_cpu_allocator();
    IAllocator* get_cuda_allocator();
    IAllocator* get_hip_allocator();
}
