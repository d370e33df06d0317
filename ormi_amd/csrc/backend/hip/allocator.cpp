// HIPAllocator: the reference's IAllocator (csrc/core/allocator.h:7-21) over
// libormi_hip, as a caching allocator.
//
// The reference's CUDAAllocator keeps exact-size free lists
// (csrc/backend/cuda/allocator.cu:36-55): a block is reused only by a request of
// the same byte count. Here requests are rounded to size classes (powers of two
// from 512 B to 1 MiB, then multiples of 2 MiB), a freed block returns to the
// cache under its real size, and a request takes the smallest cached block of
// at least its class and at most twice it. All device work is ordered on one
// stream, so a block freed by the host can be handed to the next launch at once.
// When the device is out of memory the cache is returned to it (after a
// synchronize) and the allocation retried once.
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>

#include "backend/hip/hip_backend.h"
#include "core/allocator.h"

namespace ormi {
    class HIPAllocator : public IAllocator {
        std::mutex mu_;
        std::multimap<size_t, void*> cached_;          // block size -> block
        std::unordered_map<void*, size_t> live_;       // block -> block size
        hip::AllocatorStats stats_{};

        void* take_cached(size_t cls) {
            auto it = cached_.lower_bound(cls);
            if (it == cached_.end() || it->first > 2 * cls) return nullptr;
            void* p = it->second;
            live_[p] = it->first;
            stats_.cached_bytes -= it->first;
            stats_.live_bytes += it->first;
            ++stats_.reuses;
            cached_.erase(it);
            return p;
        }

    public:
        HIPAllocator() { ORMI_HIP_CHECK(ormi_hip_init(0)); }

        void* allocate(size_t bytes) override {
            if (bytes == 0) return nullptr;
            const size_t cls = hip::size_class(bytes);
            {
                std::lock_guard<std::mutex> lock(mu_);
                if (void* p = take_cached(cls)) return p;
            }
            void* p = nullptr;
            if (ormi_hip_malloc(&p, cls) != ORMI_HIP_OK) {
                release_cached();
                ORMI_HIP_CHECK(ormi_hip_malloc(&p, cls));
            }
            std::lock_guard<std::mutex> lock(mu_);
            live_[p] = cls;
            stats_.live_bytes += cls;
            stats_.device_bytes += cls;
            ++stats_.device_mallocs;
            return p;
        }

        void free(void* ptr, size_t bytes) override {
            if (!ptr) return;
            std::lock_guard<std::mutex> lock(mu_);
            auto it = live_.find(ptr);
            const size_t sz = it != live_.end() ? it->second : hip::size_class(bytes);
            if (it != live_.end()) live_.erase(it);
            stats_.live_bytes -= sz;
            stats_.cached_bytes += sz;
            cached_.emplace(sz, ptr);
        }

        // Returns every cached block to the device. A launch error that the
        // library still holds (a queued launch that failed) is thrown after
        // the blocks are freed, so it is reported, not lost.
        void release_cached() {
            const int rc = ormi_hip_synchronize();
            const std::string msg = rc != ORMI_HIP_OK ? ormi_hip_last_error() : "";
            std::lock_guard<std::mutex> lock(mu_);
            for (auto& kv : cached_) {
                ormi_hip_free(kv.second);
                stats_.device_bytes -= kv.first;
                ++stats_.device_frees;
            }
            stats_.cached_bytes = 0;
            cached_.clear();
            if (rc != ORMI_HIP_OK) throw std::runtime_error("HIP Error: " + msg);
        }

        hip::AllocatorStats stats() {
            std::lock_guard<std::mutex> lock(mu_);
            return stats_;
        }

        void memset(void* ptr, int value, size_t bytes) override {
            ORMI_HIP_CHECK(ormi_hip_memset_d8(ptr, (unsigned char)value, bytes));
        }
        void memcpy(void* dst, const void* src, size_t size) override { ORMI_HIP_CHECK(ormi_hip_memcpy_d2d(dst, src, size)); }
        void fill_n(void* dst, const void* val, size_t elements, DType dtype) override {
            ORMI_HIP_CHECK(ormi_hip_fill(dst, val, dtype_size(dtype), elements));
        }
        void copy_device_to_host(void* dst, const void* src, size_t bytes) override {
            ORMI_HIP_CHECK(ormi_hip_memcpy_d2h(dst, src, bytes));
        }
        void copy_host_to_device(void* dst, const void* src, size_t bytes) override {
            ORMI_HIP_CHECK(ormi_hip_memcpy_h2d(dst, src, bytes));
        }
        bool is_host_visible() const override { return false; }
    };

    // Constructed on first use; a constructor that throws (no GPU) leaves the
    // HIP device unavailable, as a throwing CUDAAllocator does for CUDA.
    static HIPAllocator* hip_allocator_object() {
        static HIPAllocator* inst = new HIPAllocator();  // outlives every Buffer
        return inst;
    }
    static IAllocator* hip_allocator_instance() { return hip_allocator_object(); }
    static const bool hip_allocator_registered = (register_allocator(DeviceEnum::HIP, hip_allocator_instance), true);
}

namespace ormi::hip {
    size_t size_class(size_t bytes) {
        if (bytes <= 512) return 512;
        if (bytes <= (size_t(1) << 20)) {
            size_t c = 1024;
            while (c < bytes) c <<= 1;
            return c;
        }
        const size_t g = size_t(2) << 20;
        return (bytes + g - 1) / g * g;
    }

    AllocatorStats allocator_stats() { return hip_allocator_object()->stats(); }
    void empty_cache() { hip_allocator_object()->release_cached(); }
}
