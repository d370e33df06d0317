// HIPAllocator: the reference's IAllocator (csrc/core/allocator.h:7-21) for the
// HIP device, over libormi_hip.so. It takes the place CUDAAllocator has for
// CUDA (csrc/backend/cuda/allocator.cu:11-105), reached through the HIP case of
// get_allocator (csrc/core/allocator.cpp:5-12).
//
// Caching: CUDAAllocator reuses a block only for a request of the same byte
// count (allocator.cu:36-55). Here a request is rounded up to a size class
// (powers of two from 512 B to 1 MiB, then whole 2 MiB units) and takes the
// smallest cached block of at least that class and at most twice it, so the
// differently sized buffers of one graph share blocks. The library orders all
// device work on one stream, so a block the host frees can back the next
// launch's output at once. When the device runs out of memory the cache goes
// back to it and the allocation is retried once.
//
// fill_n's third argument is an element count, as every reference
// implementation and caller reads it (allocator.cu:69-76, csrc/core/memory.cpp:
// 100-104), although the interface names it bytes (allocator.h:15).
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>

#include "backend/hip/hip_safe_call.h"
#include "core/allocator.h"
#include "core/dtype.h"

namespace ormi {
    namespace {
        size_t size_class(size_t bytes) {
            if (bytes <= 512) return 512;
            if (bytes <= (size_t(1) << 20)) {
                size_t c = 1024;
                while (c < bytes) c <<= 1;
                return c;
            }
            const size_t unit = size_t(2) << 20;
            return (bytes + unit - 1) / unit * unit;
        }
    }

    class HIPAllocator : public IAllocator {
        std::mutex mu_;
        std::multimap<size_t, void*> cached_;     // block size -> block
        std::unordered_map<void*, size_t> live_;  // block -> block size

        // Returns every cached block to the device. A launch error the library
        // still holds is reported after the blocks are freed.
        void release_cached() {
            const int rc = ormi_hip_synchronize();
            const std::string msg = rc != ORMI_HIP_OK ? ormi_hip_last_error() : "";
            std::multimap<size_t, void*> blocks;
            {
                std::lock_guard<std::mutex> lock(mu_);
                blocks.swap(cached_);
            }
            for (auto& kv : blocks) ormi_hip_free(kv.second);
            if (rc != ORMI_HIP_OK) throw std::runtime_error("HIP Error: " + msg);
        }

    public:
        // Without a GPU ormi_hip_init fails and the constructor throws, which
        // makes the device unavailable the way a throwing CUDAAllocator does
        // (csrc/tests/test_utils.h:17-21).
        HIPAllocator() { HIP_SAFE_CALL(ormi_hip_init(0)); }

        void* allocate(size_t bytes) override {
            if (bytes == 0) return nullptr;
            const size_t cls = size_class(bytes);
            {
                std::lock_guard<std::mutex> lock(mu_);
                auto it = cached_.lower_bound(cls);
                if (it != cached_.end() && it->first <= 2 * cls) {
                    void* p = it->second;
                    live_[p] = it->first;
                    cached_.erase(it);
                    return p;
                }
            }
            void* p = nullptr;
            if (ormi_hip_malloc(&p, cls) != ORMI_HIP_OK) {
                release_cached();
                HIP_SAFE_CALL(ormi_hip_malloc(&p, cls));
            }
            std::lock_guard<std::mutex> lock(mu_);
            live_[p] = cls;
            return p;
        }

        void free(void* ptr, size_t bytes) override {
            if (!ptr) return;
            std::lock_guard<std::mutex> lock(mu_);
            auto it = live_.find(ptr);
            const size_t sz = it != live_.end() ? it->second : size_class(bytes);
            if (it != live_.end()) live_.erase(it);
            cached_.emplace(sz, ptr);
        }

        void memset(void* ptr, int value, size_t bytes) override {
            HIP_SAFE_CALL(ormi_hip_memset_d8(ptr, (unsigned char)value, bytes));
        }

        void memcpy(void* dst, const void* src, size_t size) override {
            HIP_SAFE_CALL(ormi_hip_memcpy_d2d(dst, src, size));
        }

        void fill_n(void* dst, const void* val_ptr, size_t elements, DType dtype) override {
            switch (dtype) {
                case DType::Float32:
                case DType::Int32: HIP_SAFE_CALL(ormi_hip_fill(dst, val_ptr, 4, elements)); break;
                case DType::Bool: HIP_SAFE_CALL(ormi_hip_fill(dst, val_ptr, 1, elements)); break;
                default: throw std::runtime_error("DType is not supported.");
            }
        }

        void copy_device_to_host(void* dst, const void* src, size_t bytes) override {
            HIP_SAFE_CALL(ormi_hip_memcpy_d2h(dst, src, bytes));
        }

        void copy_host_to_device(void* dst, const void* src, size_t bytes) override {
            HIP_SAFE_CALL(ormi_hip_memcpy_h2d(dst, src, bytes));
        }

        bool is_host_visible() const override { return false; }
    };

    // Built on first use and never destroyed: Buffers released during process
    // exit still find it. A constructor that throws leaves nothing behind, so
    // the next call tries again.
    IAllocator* get_hip_allocator() {
        static HIPAllocator* instance = new HIPAllocator();
        return instance;
    }
}
