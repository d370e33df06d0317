// HIP device backend (host side): allocator over the C ABI, fusion
// scheduler, hipRTC code generator, reduction and matmul graph breakers.
#pragma once
#include <cstdint>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "core/node.h"
#include "ormi_hip.h"

#define ORMI_HIP_CHECK(call)                                                                    \
    do {                                                                                        \
        int rc_ = (call);                                                                       \
        if (rc_ != ORMI_HIP_OK) throw std::runtime_error(std::string("HIP Error: ") + ormi_hip_last_error()); \
    } while (0)

namespace ormi::hip {
    using NodePtr = std::shared_ptr<Node>;

    // OpEnum -> HIP C expression over operand expressions (the reference's
    // CUDALoweringRegistry shape, csrc/backend/cuda/lowering_registry.h:11-38).
    using LoweringFunc = std::function<std::string(const std::vector<std::string>&)>;
    class HIPLoweringRegistry {
    public:
        static void register_func(ops::OpEnum op, LoweringFunc f);
        static LoweringFunc get(ops::OpEnum op);  // throws when op has no lowering
        static bool has(ops::OpEnum op);
    };

    // ---------------------------------------------------------- fusion IR --
    // A realized input of a fused kernel, with its strides aligned to the
    // kernel's logical shape (0 on broadcast dims).
    struct Leaf {
        NodePtr node;  // keeps the buffer alive until the launch is queued
        const void* ptr = nullptr;
        DType dtype = DType::Float32;
        bool scalar = false;  // 1-element buffer: read element 0 everywhere
        std::vector<long long> st;
    };

    struct Inst {
        ops::OpEnum op;
        int a = -1, b = -1;          // operand value ids
        DType cast = DType::Float32;  // CAST target
    };

    // Values 0..leaves-1 are leaves; value leaves.size()+k is insts[k].
    // roots lists the output values (one per output buffer); root == roots[0].
    struct Expr {
        std::vector<Leaf> leaves;
        std::vector<Inst> insts;
        int root = -1;
        std::vector<int> roots;
    };

    bool fusible_interior(const Node& n);
    bool fusible_root(const Node& n);
    // Most element-wise nodes one generated kernel evaluates: a longer chain is
    // cut into regions of at most this size, realized innermost first.
    constexpr size_t kMaxRegion = 256;
    // Unrealized nodes the pointwise region rooted at root reads: non-fusible
    // ones, and fusible ones beyond the region's kMaxRegion interior nodes.
    std::vector<NodePtr> region_frontier(const NodePtr& root);
    // Interior nodes of the region rooted at root, counted up to limit + 1
    // (0 when root is realized or not element-wise).
    size_t region_size(const NodePtr& root, size_t limit);
    // A reduction fuses its element-wise input as a prologue only up to this
    // many ops; a larger input is realized first, so a chain whose values feed
    // both a reduction and later element-wise ops is evaluated once, not once
    // per consumer kernel.
    constexpr size_t kMaxPrologue = 64;
    // SSA tape of the region (every frontier node must be realized), leaves
    // broadcast right-aligned to `shape`.
    // plan_only accepts realized operands of any device (kernel planning for
    // code generator tests; such an Expr is never launched).
    Expr build_expr(const NodePtr& root, const std::vector<int>& shape, bool plan_only = false);
    // One tape for several element-wise roots of the same shape: shared leaves
    // and interior nodes are evaluated once, each root is one output.
    Expr build_expr_multi(const std::vector<NodePtr>& roots, const std::vector<int>& shape, bool plan_only = false);

    // --------------------------------------------------------- kernels --
    struct FastDiv { uint32_t d, m, s; };
    FastDiv make_fastdiv(uint32_t d);

    enum class ReduceOp { Sum, Max, Argmax };

    // Summary of a launch plan (tests, debugging), formatted only on request:
    // "<kind>[ <op>] key=value ...".
    struct PlanInfo {
        const char* kind = "";
        const char* op = nullptr;
        int n = 0;
        std::pair<const char*, long long> field[10];
        void add(const char* key, long long v) {
            if (n < 10) field[n++] = {key, v};
        }
        std::string text() const;
    };

    // A generated kernel: source, entry name, launch shape, packed arguments.
    struct KernelLaunch {
        std::string source;          // empty when the kernel came from the cache
        std::string name;
        std::string key;             // structural signature (cache key)
        uint64_t handle = 0;         // compiled kernel, once known
        uint32_t grid[3] = {1, 1, 1};
        uint32_t block[3] = {256, 1, 1};
        std::vector<uint64_t> args;  // every parameter is 8 bytes
        PlanInfo plan;
    };

    // Launch-shape knobs of the generated kernels. Defaults are the values
    // measured best on MI355X; ORMI_* environment variables override them.
    struct Tuning {
        int map_unroll = 2;        // VEC groups per thread per iteration (map)
        int map_blocks_per_cu = 64;
        int row_unroll = 4;        // VEC groups per lane per iteration (row reduce)
        int col_waves = 16;        // waves per block (column reduce)
        int col_cwaves = 8;        // of those, waves side by side across the kept columns
        bool map_nt_loads = false;    // non-temporal hint on a map's operand loads
        bool map_nt_stores = true;    // non-temporal hint on a map's output stores
        bool reduce_nt_loads = true;  // non-temporal hint on a reduction's loads
        bool map_off32 = true;        // 32-bit byte offsets from uniform bases when they fit (map)
        bool map_rows = true;         // row-aligned tiles when a tile covers whole rows or lies in one (map)
    };
    const Tuning& tuning();

    // Element-wise map of expr over `shape` into out (contiguous, out_dtype).
    KernelLaunch plan_map(const Expr& expr, const std::vector<int>& shape, void* out, DType out_dtype, int compute_units);
    // The same with one contiguous output per expr.roots entry (multi-output fusion).
    KernelLaunch plan_map_multi(const Expr& expr, const std::vector<int>& shape, const std::vector<void*>& outs,
                                const std::vector<DType>& out_dtypes, int compute_units);

    // Reduction of expr (evaluated over in_shape) over `axes` (sorted; empty =
    // all). out holds prod(kept dims) values, fp32 (Sum/Max) or int64 (Argmax).
    // When the reduced range is split across work-groups, partial results go
    // to workspace (sized by reduce_workspace_bytes) and a second kernel
    // (second) finishes them.
    struct ReducePlan {
        KernelLaunch first;
        bool two_pass = false;
        KernelLaunch second;
        size_t workspace_bytes = 0;
    };
    ReducePlan plan_reduce(const Expr& expr, const std::vector<int>& in_shape, const std::vector<int>& axes, ReduceOp op,
                           void* out, int compute_units);
    void bind_workspace(ReducePlan& plan, void* workspace);

    // Source text of a planned kernel: a plan that hit the kernel cache after
    // its kernel was compiled carries only the handle, and this returns the
    // text the cache kept (diagnostics and compile-only checks).
    std::string kernel_source(const KernelLaunch& k);
    // hipRTC options every generated kernel is compiled with.
    const std::vector<std::string>& rtc_options();
    // Compile (cached) and launch.
    void launch(const KernelLaunch& k);

    // ------------------------------------------------------- scheduler --
    // Realize root on the HIP device: pointwise regions become one fused
    // kernel, reductions fuse their pointwise producer as a prologue, views
    // alias, matmuls call the MFMA GEMM.
    void realize(const NodePtr& root);
    // Realize several nodes together: element-wise roots of the same shape share
    // one multi-output kernel (each input read once); the rest realize in order.
    void realize_group(const std::vector<NodePtr>& roots);
    // Element-wise nodes run as a GEMM epilogue so far (ormi_hip_gemm_ex), and
    // the switch for that matching (on unless ORMI_GEMM_EPILOGUE=0).
    uint64_t gemm_epilogue_count();
    void set_gemm_epilogue(bool on);

    // ------------------------------------------------------- allocator --
    struct AllocatorStats {
        size_t live_bytes = 0;      // in blocks handed out
        size_t cached_bytes = 0;    // in blocks waiting for reuse
        size_t device_bytes = 0;    // held from the device (live + cached)
        uint64_t device_mallocs = 0;
        uint64_t device_frees = 0;
        uint64_t reuses = 0;        // requests served from the cache
    };
    // Bytes a request of `bytes` occupies: powers of two from 512 B to 1 MiB,
    // then multiples of 2 MiB.
    size_t size_class(size_t bytes);
    AllocatorStats allocator_stats();  // throws when the HIP device is absent
    void empty_cache();                // return every cached block to the device
    int device_compute_units();
}
