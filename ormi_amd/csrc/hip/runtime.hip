// libormi_hip.so: device set-up, memory, hipRTC compile cache, kernel launch,
// events, and the small fill/convert kernels. Implements include/ormi_hip.h.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <thread>
#include <string>
#include <unordered_map>
#include <vector>

// The architecture the library is built for (set by the build; gfx950).
#ifndef ORMI_HIP_TARGET
#define ORMI_HIP_TARGET "gfx950"
#endif

#include "ormi_hip.h"
#include "ormi_hip_internal.h"
#include "device/ormi_device.h"

namespace ormi_hip {

static thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

struct DeviceState {
    std::mutex mu;
    bool inited = false;
    int device = -1;
    hipDeviceProp_t props{};
    std::string arch;  // full target id, e.g. gfx950:sramecc+:xnack-
};

static DeviceState& state() {
    static DeviceState* s = new DeviceState();  // never destroyed: buffers may be freed at exit
    return *s;
}

int ensure_init() {
    DeviceState& s = state();
    if (s.inited) return ORMI_HIP_OK;
    return ormi_hip_init(0);
}

int compute_units() {
    return state().inited ? state().props.multiProcessorCount : 256;
}

// ---------------------------------------------------------------- kernels --
template <typename T>
__global__ void fill_kernel(T* __restrict__ dst, T value, size_t count) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) dst[i] = value;
}

__device__ __forceinline__ float load_as_f32(const void* p, int dt, size_t i) {
    switch (dt) {
        case ORMI_DTYPE_F32: return ((const float*)p)[i];
        case ORMI_DTYPE_BF16: return ormi_bf16_to_f32(((const unsigned short*)p)[i]);
        case ORMI_DTYPE_F16: return ormi_f16_to_f32(((const unsigned short*)p)[i]);
        case ORMI_DTYPE_I32: return (float)((const int*)p)[i];
        case ORMI_DTYPE_I64: return (float)((const long long*)p)[i];
        default: return ((const unsigned char*)p)[i] ? 1.0f : 0.0f;
    }
}

__device__ __forceinline__ bool is_int_dtype(int dt) {
    return dt == ORMI_DTYPE_I32 || dt == ORMI_DTYPE_I64 || dt == ORMI_DTYPE_BOOL;
}

__device__ __forceinline__ long long load_as_i64(const void* p, int dt, size_t i) {
    switch (dt) {
        case ORMI_DTYPE_I32: return ((const int*)p)[i];
        case ORMI_DTYPE_I64: return ((const long long*)p)[i];
        default: return ((const unsigned char*)p)[i] ? 1 : 0;
    }
}

// dst[i] = src[i] as dst's dtype. Between integer types (bool included) the
// value converts exactly, an int64 outside the int32 range saturating and a
// nonzero value giving true; from a float type it goes through float32 (the
// ormi_f32_to_* rules: truncation, NaN to 0, saturation); to a float type it
// rounds to nearest even.
__global__ void convert_kernel(void* __restrict__ dst, int dst_dt, const void* __restrict__ src, int src_dt, size_t count) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const bool int_to_int = is_int_dtype(src_dt) && is_int_dtype(dst_dt);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        if (int_to_int) {
            const long long v = load_as_i64(src, src_dt, i);
            switch (dst_dt) {
                case ORMI_DTYPE_I64: ((long long*)dst)[i] = v; break;
                case ORMI_DTYPE_I32: ((int*)dst)[i] = v > 2147483647LL ? 2147483647 : v < -2147483648LL ? (int)0x80000000u : (int)v; break;
                default: ((unsigned char*)dst)[i] = v != 0; break;
            }
            continue;
        }
        const float v = load_as_f32(src, src_dt, i);
        switch (dst_dt) {
            case ORMI_DTYPE_F32: ((float*)dst)[i] = v; break;
            case ORMI_DTYPE_BF16: ((unsigned short*)dst)[i] = ormi_f32_to_bf16(v); break;
            case ORMI_DTYPE_F16: ((unsigned short*)dst)[i] = ormi_f32_to_f16(v); break;
            case ORMI_DTYPE_I32: ((int*)dst)[i] = ormi_f32_to_i32(v); break;
            case ORMI_DTYPE_I64: ((long long*)dst)[i] = ormi_f32_to_i64(v); break;
            default: ((unsigned char*)dst)[i] = v != 0.0f; break;
        }
    }
}

static unsigned grid_for(size_t count, unsigned block) {
    size_t g = (count + block - 1) / block;
    const size_t cap = (size_t)compute_units() * 8;
    if (g > cap) g = cap;
    return g ? (unsigned)g : 1u;
}

// ------------------------------------------------------------ rtc cache --
struct RtcEntry {
    hipModule_t module;
    hipFunction_t function;
};

struct RtcCache {
    std::mutex mu;
    std::unordered_map<std::string, uint64_t> by_key;
    std::vector<RtcEntry> entries;
};

static RtcCache& rtc_cache() {
    static RtcCache* c = new RtcCache();
    return *c;
}

static int rtc_build(const char* source, const std::string& target, const char* const* options, int num_options,
                     std::vector<char>& code) {
    hiprtcProgram prog;
    hiprtcResult r = hiprtcCreateProgram(&prog, source, "ormi_generated.hip", 0, nullptr, nullptr);
    if (r != HIPRTC_SUCCESS) return fail(ORMI_HIP_ERR_COMPILE, std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
    std::vector<std::string> opts;
    opts.push_back("--offload-arch=" + target);
    for (int i = 0; i < num_options; ++i) opts.emplace_back(options[i]);
    std::vector<const char*> copts;
    for (auto& o : opts) copts.push_back(o.c_str());
    r = hiprtcCompileProgram(prog, (int)copts.size(), copts.data());
    if (r != HIPRTC_SUCCESS) {
        size_t log_size = 0;
        hiprtcGetProgramLogSize(prog, &log_size);
        std::string log(log_size + 1, '\0');
        if (log_size) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        return fail(ORMI_HIP_ERR_COMPILE, std::string("hipRTC compile failed: ") + hiprtcGetErrorString(r) + "\n" + log);
    }
    size_t code_size = 0;
    hiprtcGetCodeSize(prog, &code_size);
    code.resize(code_size);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    return ORMI_HIP_OK;
}

// ---------------------------------------------------------- upload ring --
// Host-to-device copies are stream-ordered, not synchronous: the bytes are
// copied into a pinned ring and an asynchronous copy from there is enqueued on
// the null stream, so an upload neither waits for the kernels before it nor
// blocks the host while the DMA runs. The caller's buffer is free on return.
// Each enqueued piece records an event; a piece that would overwrite ring
// bytes an earlier copy has not read yet waits on the newest such copy's
// event (the stream is in order, so every older copy is then done as well).
// Uploads larger than one piece go through in PIECE-sized parts, the host
// copy of a part overlapping the DMA of the one before.
struct UploadRing {
    static constexpr size_t RING = 64u << 20;   // pinned bytes
    static constexpr size_t PIECE = 16u << 20;  // largest single copy
    static constexpr size_t ALIGN = 256;
    static constexpr size_t MAX_PENDING = 4096;  // enqueued pieces not yet known complete
    struct Region {
        size_t beg, end;
        hipEvent_t ev;
    };
    std::mutex mu;
    char* base = nullptr;
    bool unavailable = false;  // pinned allocation failed: copies are synchronous
    size_t head = 0;
    std::deque<Region> pending;  // in enqueue order
    std::vector<hipEvent_t> spare;

    int event(hipEvent_t* ev) {
        if (!spare.empty()) {
            *ev = spare.back();
            spare.pop_back();
            return ORMI_HIP_OK;
        }
        const hipError_t e = hipEventCreateWithFlags(ev, hipEventDisableTiming);
        if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("upload ring: hipEventCreate: ") + hipGetErrorString(e));
        return ORMI_HIP_OK;
    }
    void retire(size_t count) {  // the oldest count entries are complete
        for (; count > 0; --count) {
            spare.push_back(pending.front().ev);
            pending.pop_front();
        }
    }
    // Position of n bytes (n <= PIECE) that no pending copy still reads.
    int reserve(size_t n, size_t* pos) {
        size_t p = (head + ALIGN - 1) / ALIGN * ALIGN;
        if (p + n > RING) p = 0;
        // Completed entries at the front need no wait.
        while (!pending.empty() && hipEventQuery(pending.front().ev) == hipSuccess) retire(1);
        size_t last = SIZE_MAX;
        for (size_t i = 0; i < pending.size(); ++i)
            if (pending[i].beg < p + n && p < pending[i].end) last = i;
        if (last == SIZE_MAX && pending.size() >= MAX_PENDING) last = 0;
        if (last != SIZE_MAX) {
            const hipError_t e = hipEventSynchronize(pending[last].ev);
            if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("upload ring: hipEventSynchronize: ") + hipGetErrorString(e));
            retire(last + 1);
        }
        *pos = p;
        head = p + n;
        return ORMI_HIP_OK;
    }
    int upload(char* dst, const char* src, size_t bytes) {
        std::lock_guard<std::mutex> lock(mu);
        if (!base && !unavailable) {
            if (hipHostMalloc((void**)&base, RING, hipHostMallocDefault) != hipSuccess) {
                base = nullptr;
                unavailable = true;
                (void)hipGetLastError();
            }
        }
        if (unavailable) {
            const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
            if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("hipMemcpy: ") + hipGetErrorString(e));
            return ORMI_HIP_OK;
        }
        for (size_t off = 0; off < bytes; off += PIECE) {
            const size_t n = bytes - off < PIECE ? bytes - off : PIECE;
            size_t p;
            int rc = reserve(n, &p);
            if (rc != ORMI_HIP_OK) return rc;
            std::memcpy(base + p, src + off, n);
            hipEvent_t ev;
            if ((rc = event(&ev)) != ORMI_HIP_OK) return rc;
            hipError_t e = hipMemcpyAsync(dst + off, base + p, n, hipMemcpyHostToDevice, 0);
            if (e != hipSuccess) {
                spare.push_back(ev);
                return fail(ORMI_HIP_ERR_RUNTIME, std::string("upload ring: hipMemcpyAsync: ") + hipGetErrorString(e));
            }
            e = hipEventRecord(ev, 0);
            if (e != hipSuccess) {
                // The copy is queued but untracked: wait for it, so no later
                // piece overwrites ring bytes it has not read yet.
                spare.push_back(ev);
                (void)hipStreamSynchronize(0);
                return fail(ORMI_HIP_ERR_RUNTIME, std::string("upload ring: hipEventRecord: ") + hipGetErrorString(e));
            }
            pending.push_back({p, p + n, ev});
        }
        return ORMI_HIP_OK;
    }
};

static UploadRing& upload_ring() {
    static UploadRing* r = new UploadRing();  // never destroyed: pinned memory lives until exit
    return *r;
}

// ----------------------------------------------------------- launch queue --
// Launches of generated kernels (ormi_hip_launch_queued) are recorded here and
// issued to the null stream, in submission order, by one worker thread. A HIP
// launch costs the calling thread about 3.5 us on MI355X hosts whatever its
// form, more than a small fused kernel runs; with the queue the thread that
// builds graphs pays a copy of the arguments instead, and launching overlaps
// its next graph. Every other entry point that touches the device first waits
// until the queue has issued everything submitted before it (drain_queue), so
// the stream sees exactly the order of the calls, as without the queue.
struct QueuedLaunch {
    hipFunction_t fn;
    uint32_t grid[3], block[3], lds;
    int nargs;
    uint64_t args[ORMI_HIP_QUEUED_MAX_ARGS];
};

struct LaunchQueue {
    static constexpr uint64_t N = 1024;
    QueuedLaunch slot[N];
    std::atomic<uint64_t> head{0};  // submitted
    std::atomic<uint64_t> tail{0};  // issued
    std::mutex submit_mu;           // one submitter at a time
    std::mutex sleep_mu;
    std::condition_variable wake;
    std::atomic<bool> sleeping{false};
    std::atomic<bool> stop{false};
    std::atomic<bool> failed{false};
    std::mutex err_mu;
    std::string error;
    std::thread worker;
    bool started = false;
    int device = 0;

    void run() {
        if (hipSetDevice(device) != hipSuccess) {
            record_error("launch queue: hipSetDevice failed");
        }
        for (;;) {
            const uint64_t t = tail.load(std::memory_order_relaxed);
            if (head.load(std::memory_order_acquire) == t) {
                if (stop.load()) return;
                // Spin (yielding) for kSpin after the last launch, then sleep:
                // launches come in bursts separated by host work (building the
                // next graph, a training step's Python), and a launch that has
                // to wake a sleeping worker waits tens of microseconds for it.
                constexpr auto kSpin = std::chrono::microseconds(2000);
                const auto spin_end = std::chrono::steady_clock::now() + kSpin;
                bool got = false;
                for (int i = 0; !got; ++i) {
                    if (head.load(std::memory_order_acquire) != t) got = true;
                    else if ((i & 63) == 63) {
                        if (std::chrono::steady_clock::now() >= spin_end) break;
                        std::this_thread::yield();
                    }
                }
                if (!got) {
                    std::unique_lock<std::mutex> lock(sleep_mu);
                    sleeping.store(true);
                    wake.wait(lock, [&] { return head.load() != t || stop.load(); });
                    sleeping.store(false);
                }
                continue;
            }
            QueuedLaunch& q = slot[t % N];
            void* ptrs[ORMI_HIP_QUEUED_MAX_ARGS];
            for (int i = 0; i < q.nargs; ++i) ptrs[i] = &q.args[i];
            const hipError_t e = hipModuleLaunchKernel(q.fn, q.grid[0], q.grid[1], q.grid[2], q.block[0], q.block[1],
                                                       q.block[2], q.lds, 0, ptrs, nullptr);
            if (e != hipSuccess) record_error(std::string("queued kernel launch: ") + hipGetErrorString(e));
            tail.store(t + 1, std::memory_order_release);
        }
    }
    void record_error(const std::string& msg) {
        std::lock_guard<std::mutex> lock(err_mu);
        if (!failed.load()) error = msg;
        failed.store(true);
    }
};

static LaunchQueue& launch_queue() {
    static LaunchQueue* q = new LaunchQueue();  // never destroyed: the worker is joined at exit
    return *q;
}

static void stop_launch_queue() {
    LaunchQueue& q = launch_queue();
    if (!q.started) return;
    q.stop.store(true);
    {
        std::lock_guard<std::mutex> lock(q.sleep_mu);
        q.wake.notify_all();
    }
    q.worker.join();
    q.started = false;
}

// Wait until every queued launch has been issued; report a failed one.
int drain_queue() {
    LaunchQueue& q = launch_queue();
    if (q.started) {
        while (q.tail.load(std::memory_order_acquire) != q.head.load(std::memory_order_acquire)) std::this_thread::yield();
    }
    if (q.failed.load()) {
        std::lock_guard<std::mutex> lock(q.err_mu);
        q.failed.store(false);
        return fail(ORMI_HIP_ERR_RUNTIME, q.error);
    }
    return ORMI_HIP_OK;
}

static int submit_launch(hipFunction_t fn, const uint32_t grid[3], const uint32_t block[3], uint32_t lds,
                         const uint64_t* args, int nargs) {
    LaunchQueue& q = launch_queue();
    std::lock_guard<std::mutex> lock(q.submit_mu);
    if (q.failed.load()) {  // an earlier queued launch failed: report it here, as the next call
        std::lock_guard<std::mutex> el(q.err_mu);
        q.failed.store(false);
        return fail(ORMI_HIP_ERR_RUNTIME, q.error);
    }
    if (!q.started) {
        q.device = state().device;
        q.worker = std::thread([&q] { q.run(); });
        q.started = true;
        std::atexit(stop_launch_queue);
    }
    const uint64_t h = q.head.load(std::memory_order_relaxed);
    while (h - q.tail.load(std::memory_order_acquire) >= LaunchQueue::N) std::this_thread::yield();
    QueuedLaunch& s = q.slot[h % LaunchQueue::N];
    s.fn = fn;
    for (int i = 0; i < 3; ++i) {
        s.grid[i] = grid[i];
        s.block[i] = block[i];
    }
    s.lds = lds;
    s.nargs = nargs;
    std::memcpy(s.args, args, sizeof(uint64_t) * (size_t)nargs);
    q.head.store(h + 1, std::memory_order_seq_cst);
    if (q.sleeping.load(std::memory_order_seq_cst)) {
        std::lock_guard<std::mutex> sl(q.sleep_mu);
        q.wake.notify_one();
    }
    return ORMI_HIP_OK;
}

}  // namespace ormi_hip

using namespace ormi_hip;

#define ORMI_HIP_TRY(call)                                                                           \
    do {                                                                                             \
        hipError_t e_ = (call);                                                                      \
        if (e_ != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define ORMI_ENSURE_INIT()                    \
    do {                                      \
        int rc_ = ensure_init();              \
        if (rc_ != ORMI_HIP_OK) return rc_;   \
    } while (0)

// Issue every queued launch first (stream order; see the launch queue).
#define ORMI_HIP_DRAIN()                      \
    do {                                      \
        int rc_ = drain_queue();              \
        if (rc_ != ORMI_HIP_OK) return rc_;   \
    } while (0)

extern "C" {

const char* ormi_hip_last_error(void) { return g_last_error.c_str(); }

int ormi_hip_device_count(int* count) {
    if (!count) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_device_count: null output");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
    return ORMI_HIP_OK;
}

int ormi_hip_init(int device) {
    DeviceState& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (s.inited) {
        if (device != s.device) return fail(ORMI_HIP_ERR_UNSUPPORTED, "ormi_hip_init: library already bound to another device");
        return ORMI_HIP_OK;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(ORMI_HIP_ERR_NO_DEVICE, "HIP Error: no GPU device is visible to this process");
    if (device < 0 || device >= n) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_init: device index out of range");
    hipDeviceProp_t props;
    ORMI_HIP_TRY(hipGetDeviceProperties(&props, device));
    // The precompiled kernels exist for the build's target only, and the
    // generated kernels' launch shapes assume gfx950's 160 KB of LDS per CU.
    const size_t tn = std::strlen(ORMI_HIP_TARGET);
    if (std::strncmp(props.gcnArchName, ORMI_HIP_TARGET, tn) != 0 ||
        (props.gcnArchName[tn] != '\0' && props.gcnArchName[tn] != ':'))
        return fail(ORMI_HIP_ERR_UNSUPPORTED, std::string("ormi_hip_init: this library is built for ") + ORMI_HIP_TARGET +
                                                  "; device " + std::to_string(device) + " is " + props.gcnArchName);
    ORMI_HIP_TRY(hipSetDevice(device));
    s.props = props;
    const int rc = gemm_scratch_setup();
    if (rc != ORMI_HIP_OK) return rc;
    s.arch = s.props.gcnArchName;
    s.device = device;
    s.inited = true;
    return ORMI_HIP_OK;
}

int ormi_hip_get_props(ormi_hip_props* out) {
    if (!out) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_get_props: null output");
    ORMI_ENSURE_INIT();
    const DeviceState& s = state();
    std::memset(out, 0, sizeof(*out));
    std::strncpy(out->name, s.arch.c_str(), sizeof(out->name) - 1);
    out->compute_units = s.props.multiProcessorCount;
    out->clock_khz = s.props.clockRate;
    out->lds_bytes_per_block = (int)s.props.sharedMemPerBlock;
    out->total_mem_bytes = s.props.totalGlobalMem;
    return ORMI_HIP_OK;
}

int ormi_hip_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_malloc: null output");
    ORMI_ENSURE_INIT();
    *ptr = nullptr;
    if (bytes == 0) return ORMI_HIP_OK;
    ORMI_HIP_TRY(hipMalloc(ptr, bytes));
    return ORMI_HIP_OK;
}

// The block is freed even when a queued launch failed (the error of that
// launch is returned afterwards), so the failure does not leak it.
int ormi_hip_free(void* ptr) {
    if (!ptr) return ORMI_HIP_OK;
    const int queued = drain_queue();
    const std::string queued_msg = queued != ORMI_HIP_OK ? g_last_error : std::string();
    ORMI_HIP_TRY(hipFree(ptr));
    if (queued != ORMI_HIP_OK) return fail(queued, queued_msg);
    return ORMI_HIP_OK;
}

int ormi_hip_fill(void* dst, const void* value, size_t elem_bytes, size_t count) {
    if (count == 0) return ORMI_HIP_OK;
    if (!dst || !value) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_fill: null pointer");
    ORMI_ENSURE_INIT();
    ORMI_HIP_DRAIN();
    const unsigned block = 256, grid = grid_for(count, block);
    switch (elem_bytes) {
        case 1: { unsigned char v; std::memcpy(&v, value, 1); fill_kernel<unsigned char><<<grid, block>>>((unsigned char*)dst, v, count); break; }
        case 2: { unsigned short v; std::memcpy(&v, value, 2); fill_kernel<unsigned short><<<grid, block>>>((unsigned short*)dst, v, count); break; }
        case 4: { unsigned v; std::memcpy(&v, value, 4); fill_kernel<unsigned><<<grid, block>>>((unsigned*)dst, v, count); break; }
        case 8: { unsigned long long v; std::memcpy(&v, value, 8); fill_kernel<unsigned long long><<<grid, block>>>((unsigned long long*)dst, v, count); break; }
        default: return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_fill: element size must be 1, 2, 4 or 8");
    }
    ORMI_HIP_TRY(hipGetLastError());
    return ORMI_HIP_OK;
}

int ormi_hip_memset_d8(void* dst, unsigned char value, size_t count) { return ormi_hip_fill(dst, &value, 1, count); }
int ormi_hip_memset_d32(void* dst, uint32_t value, size_t count) { return ormi_hip_fill(dst, &value, 4, count); }

int ormi_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return ORMI_HIP_OK;
    if (!dst || !src) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_memcpy_h2d: null pointer");
    ORMI_ENSURE_INIT();
    ORMI_HIP_DRAIN();
    return upload_ring().upload((char*)dst, (const char*)src, bytes);
}

int ormi_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return ORMI_HIP_OK;
    if (!dst || !src) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_memcpy_d2h: null pointer");
    ORMI_ENSURE_INIT();
    ORMI_HIP_DRAIN();
    ORMI_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return ORMI_HIP_OK;
}

int ormi_hip_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return ORMI_HIP_OK;
    if (!dst || !src) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_memcpy_d2d: null pointer");
    ORMI_ENSURE_INIT();
    ORMI_HIP_DRAIN();
    ORMI_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, 0));
    return ORMI_HIP_OK;
}

int ormi_hip_synchronize(void) {
    ORMI_ENSURE_INIT();
    ORMI_HIP_DRAIN();
    ORMI_HIP_TRY(hipDeviceSynchronize());
    return ORMI_HIP_OK;
}

int ormi_hip_convert(void* dst, int dst_dtype, const void* src, int src_dtype, size_t count) {
    if (count == 0) return ORMI_HIP_OK;
    if (!dst || !src) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_convert: null pointer");
    if (dst_dtype < 0 || dst_dtype > ORMI_DTYPE_I64 || src_dtype < 0 || src_dtype > ORMI_DTYPE_I64)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_convert: unknown dtype code");
    ORMI_ENSURE_INIT();
    ORMI_HIP_DRAIN();
    const unsigned block = 256, grid = grid_for(count, block);
    convert_kernel<<<grid, block>>>(dst, dst_dtype, src, src_dtype, count);
    ORMI_HIP_TRY(hipGetLastError());
    return ORMI_HIP_OK;
}

int ormi_hip_rtc_compile(const char* source, const char* kernel_name, const char* const* options, int num_options,
                         uint64_t* handle) {
    if (!source || !kernel_name || !handle || (num_options > 0 && !options))
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_rtc_compile: null argument");
    ORMI_ENSURE_INIT();
    std::string key(kernel_name);
    key.push_back('\0');
    for (int i = 0; i < num_options; ++i) {
        key += options[i];
        key.push_back('\0');
    }
    key += source;
    RtcCache& c = rtc_cache();
    {
        std::lock_guard<std::mutex> lock(c.mu);
        auto it = c.by_key.find(key);
        if (it != c.by_key.end()) {
            *handle = it->second;
            return ORMI_HIP_OK;
        }
    }
    std::vector<char> code;
    int rc = rtc_build(source, state().arch, options, num_options, code);
    if (rc != ORMI_HIP_OK) return rc;
    RtcEntry e{};
    ORMI_HIP_TRY(hipModuleLoadData(&e.module, code.data()));
    hipError_t ge = hipModuleGetFunction(&e.function, e.module, kernel_name);
    if (ge != hipSuccess) {
        (void)hipModuleUnload(e.module);
        return fail(ORMI_HIP_ERR_COMPILE, std::string("hipModuleGetFunction(") + kernel_name + "): " + hipGetErrorString(ge));
    }
    std::lock_guard<std::mutex> lock(c.mu);
    auto it = c.by_key.find(key);
    if (it != c.by_key.end()) {  // another thread compiled the same source meanwhile
        (void)hipModuleUnload(e.module);
        *handle = it->second;
        return ORMI_HIP_OK;
    }
    c.entries.push_back(e);
    *handle = (uint64_t)c.entries.size();
    c.by_key.emplace(std::move(key), *handle);
    return ORMI_HIP_OK;
}

int ormi_hip_rtc_compile_only(const char* source, const char* target, const char* const* options, int num_options,
                              size_t* code_bytes) {
    if (!source || !target || !code_bytes || (num_options > 0 && !options))
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_rtc_compile_only: null argument");
    std::vector<char> code;
    int rc = rtc_build(source, target, options, num_options, code);
    if (rc != ORMI_HIP_OK) return rc;
    *code_bytes = code.size();
    return ORMI_HIP_OK;
}

int ormi_hip_rtc_cache_size(uint64_t* entries) {
    if (!entries) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_rtc_cache_size: null output");
    RtcCache& c = rtc_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    *entries = c.entries.size();
    return ORMI_HIP_OK;
}

int ormi_hip_launch(uint64_t handle, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes, void** args) {
    if (!grid || !block) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_launch: null grid/block");
    hipFunction_t fn;
    {
        RtcCache& c = rtc_cache();
        std::lock_guard<std::mutex> lock(c.mu);
        if (handle == 0 || handle > c.entries.size()) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_launch: unknown kernel handle");
        fn = c.entries[handle - 1].function;
    }
    if (grid[0] == 0 || grid[1] == 0 || grid[2] == 0) return ORMI_HIP_OK;  // empty launch: nothing to do
    if (block[0] * block[1] * block[2] == 0 || block[0] * block[1] * block[2] > 1024)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_launch: block size must be 1..1024 threads");
    ORMI_HIP_DRAIN();
    ORMI_HIP_TRY(hipModuleLaunchKernel(fn, grid[0], grid[1], grid[2], block[0], block[1], block[2], lds_bytes, 0, args, nullptr));
    return ORMI_HIP_OK;
}

int ormi_hip_launch_queued(uint64_t handle, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes,
                           const uint64_t* args, int num_args) {
    if (!grid || !block || (num_args > 0 && !args)) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_launch_queued: null argument");
    if (num_args < 0 || num_args > ORMI_HIP_QUEUED_MAX_ARGS)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_launch_queued: more than ORMI_HIP_QUEUED_MAX_ARGS arguments");
    hipFunction_t fn;
    {
        RtcCache& c = rtc_cache();
        std::lock_guard<std::mutex> lock(c.mu);
        if (handle == 0 || handle > c.entries.size()) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_launch_queued: unknown kernel handle");
        fn = c.entries[handle - 1].function;
    }
    if (grid[0] == 0 || grid[1] == 0 || grid[2] == 0) return ORMI_HIP_OK;
    if (block[0] * block[1] * block[2] == 0 || block[0] * block[1] * block[2] > 1024)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_launch_queued: block size must be 1..1024 threads");
    return submit_launch(fn, grid, block, lds_bytes, args, num_args);
}

// Test hook, outside the C ABI of include/ormi_hip.h: records msg as the error
// of a queued launch, exactly as the launch thread records a launch the runtime
// refused, so a test can check that the next call reports it without making a
// launch fail on the device. Touches no device state.
__attribute__((visibility("default"))) int ormi_hip_test_fail_queued_launch(const char* msg) {
    launch_queue().record_error(std::string("queued kernel launch: ") + (msg ? msg : ""));
    return ORMI_HIP_OK;
}

int ormi_hip_event_create(void** event) {
    if (!event) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_event_create: null output");
    ORMI_ENSURE_INIT();
    hipEvent_t e;
    ORMI_HIP_TRY(hipEventCreate(&e));
    *event = (void*)e;
    return ORMI_HIP_OK;
}

int ormi_hip_event_record(void* event) {
    if (!event) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_event_record: null event");
    ORMI_HIP_DRAIN();
    ORMI_HIP_TRY(hipEventRecord((hipEvent_t)event, 0));
    return ORMI_HIP_OK;
}

int ormi_hip_event_elapsed_ms(void* start, void* end, float* ms) {
    if (!start || !end || !ms) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_event_elapsed_ms: null argument");
    ORMI_HIP_TRY(hipEventSynchronize((hipEvent_t)end));
    ORMI_HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
    return ORMI_HIP_OK;
}

int ormi_hip_event_destroy(void* event) {
    if (!event) return ORMI_HIP_OK;
    ORMI_HIP_TRY(hipEventDestroy((hipEvent_t)event));
    return ORMI_HIP_OK;
}

}  // extern "C"
