#include <stdexcept>
#include <map>
#include <mutex>
#include "core/allocator.h"

namespace ormi {
    static std::map<DeviceEnum, AllocatorGetter>& allocator_table() {
        static std::map<DeviceEnum, AllocatorGetter> table;
        return table;
    }
    static std::mutex& table_mutex() { static std::mutex m; return m; }

    void register_allocator(DeviceEnum dev, AllocatorGetter getter) {
        std::lock_guard<std::mutex> lock(table_mutex());
        allocator_table()[dev] = getter;
    }

    bool has_allocator(DeviceEnum dev) {
        std::lock_guard<std::mutex> lock(table_mutex());
        return allocator_table().count(dev) > 0;
    }

    IAllocator* get_allocator(DeviceEnum type) {
        AllocatorGetter getter = nullptr;
        {
            std::lock_guard<std::mutex> lock(table_mutex());
            auto it = allocator_table().find(type);
            if (it != allocator_table().end()) getter = it->second;
        }
        if (!getter) {
            if (type == DeviceEnum::CPU)
                throw std::runtime_error("Unsupported DeviceEnum: no CPU backend is loaded in this process (this library provides the HIP device).");
            if (type == DeviceEnum::CUDA)
                throw std::runtime_error("Unsupported DeviceEnum: this library has no CUDA backend.");
            throw std::runtime_error("Unsupported DeviceEnum.");
        }
        return getter();
    }

    IAllocator* get_cpu_allocator() { return get_allocator(DeviceEnum::CPU); }
    IAllocator* get_cuda_allocator() { return get_allocator(DeviceEnum::CUDA); }
    IAllocator* get_hip_allocator() { return get_allocator(DeviceEnum::HIP); }
}
