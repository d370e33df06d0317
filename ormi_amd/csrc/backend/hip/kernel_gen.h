// Kernel IR of the hipRTC code generator and the generator's interface.
// Depends on the dtype and op enums only (no graph types), so the generator is
// built twice: into the host core, where the fusion scheduler feeds it, and
// into the device layer libormi_hip.so, where ormi_hip_reduce feeds it a plain
// strided input and ormi_hip_map a caller's tape. Both emit the same kernels
// for the same request.
#pragma once
#include <cstdint>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "core/dtype.h"
#include "core/ops.h"
#include "ormi_hip.h"

#define ORMI_HIP_CHECK(call)                                                                    \
    do {                                                                                        \
        int rc_ = (call);                                                                       \
        if (rc_ != ORMI_HIP_OK) throw std::runtime_error(std::string("HIP Error: ") + ormi_hip_last_error()); \
    } while (0)

namespace ormi::hip {
    // Operand expressions -> HIP C expression of one op (the reference's
    // CUDALoweringRegistry shape, csrc/backend/cuda/lowering_registry.h:11-38).
    using LoweringFunc = std::function<std::string(const std::vector<std::string>&)>;
    // The built-in lowering of an element-wise op (device functions of
    // ormi_device.h), or nullptr for an op without one (CAST is lowered by the
    // generator itself). Every path that builds a tape takes its lowerings from
    // here, so the same tape gives the same kernel text.
    const LoweringFunc* builtin_lowering(ops::OpEnum op);

    // ---------------------------------------------------------- fusion IR --
    // A realized input of a fused kernel, with its strides aligned to the
    // kernel's logical shape (0 on broadcast dims).
    struct Leaf {
        std::shared_ptr<const void> keep;  // keeps the buffer alive until the launch is queued
        const void* ptr = nullptr;
        DType dtype = DType::Float32;
        bool scalar = false;  // 1-element buffer: read element 0 everywhere
        std::vector<long long> st;
    };

    struct Inst {
        ops::OpEnum op;
        int a = -1, b = -1;          // operand value ids
        DType cast = DType::Float32;  // CAST target
        const LoweringFunc* lower = nullptr;  // C expression of op (every op but CAST)
    };

    // Values 0..leaves-1 are leaves; value leaves.size()+k is insts[k].
    // roots lists the output values (one per output buffer); root == roots[0].
    struct Expr {
        std::vector<Leaf> leaves;
        std::vector<Inst> insts;
        int root = -1;
        std::vector<int> roots;
    };

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
        // Dynamic LDS per work-group, allocated at launch and never touched by
        // the kernel: it caps the work-groups resident per CU (see
        // Tuning::map_wg_per_cu).
        uint32_t lds = 0;
        std::vector<uint64_t> args;  // every parameter is 8 bytes
        PlanInfo plan;
        // Arguments that hold a buffer address, as (argument index, source):
        // source >= 0 is that leaf's pointer, -1 - r is output r. A repeat
        // request reuses the plan and rewrites only these.
        std::vector<std::pair<int, int>> ptr_slots;
    };

    // Launch-shape knobs of the generated kernels. Defaults are the values
    // measured best on MI355X; ORMI_* environment variables override them.
    struct Tuning {
        int map_unroll = 2;        // VEC groups per thread per iteration (map)
        int map_blocks_per_cu = 64;
        int row_unroll = 4;        // VEC groups per lane per iteration (row reduce)
        int row_waves = 4;         // waves sharing one long row (row reduce; 1, 2 or 4)
        int row_waves_min_groups = 1024;  // row length (VEC groups) from which rows are shared
        int col_waves = 16;        // waves per block (column reduce)
        int col_cwaves = 16;       // of those, waves side by side across the kept columns
        int col_unroll = 2;        // rows in flight per wave (column reduce)
        int col_fin_split = 4;     // lanes per column in a column sum's finish pass (1, 2, 4 or 8)
        // Work-groups resident per CU for map / row-reduction kernels whose grid
        // would hold more (0: no cap). HBM streams run faster with fewer
        // concurrent ones: see occupancy_lds.
        int map_wg_per_cu = 5;
        int map_row_tile_wg_per_cu = 6;  // the same for maps on tiles of several rows (bias rows)
        int row_wg_per_cu = 3;      // row sums
        int row_max_wg_per_cu = 4;  // row max / argmax: a longer dependent chain per element
        bool map_nt_loads = true;     // non-temporal hint on a map's operand loads
        bool map_nt_stores = true;    // non-temporal hint on a map's output stores
        bool reduce_nt_loads = true;  // non-temporal hint on a reduction's loads
        // Both load hints apply only to leaves read once (no broadcast), in
        // kernels whose such leaves bring in at least this many bytes.
        long long nt_min_bytes = 64LL << 20;
        bool map_off32 = true;        // 32-bit byte offsets from uniform bases when they fit (map)
        bool map_rows = true;         // row-aligned tiles when a tile covers whole rows or lies in one (map)
        bool map_row_tiles = true;    // tiles of `unroll` rows x 256 groups when an operand is a bias row (map)
    };
    const Tuning& tuning();

    // Element-wise map of expr over `shape` into out (contiguous, out_dtype).
    // launch_only: the caller only launches the result, so a repeat request
    // whose kernel is compiled returns just the handle, launch shape and
    // arguments (no name, signature or plan text to copy).
    KernelLaunch plan_map(const Expr& expr, const std::vector<int>& shape, void* out, DType out_dtype, int compute_units,
                          bool launch_only = false);
    // The same with one contiguous output per expr.roots entry (multi-output fusion).
    KernelLaunch plan_map_multi(const Expr& expr, const std::vector<int>& shape, const std::vector<void*>& outs,
                                const std::vector<DType>& out_dtypes, int compute_units, bool launch_only = false);

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
    // An element-wise consumer of a Sum or Max result, applied as the result
    // is stored (the mean's 1/N, a scaled or shifted sum), so it needs no
    // kernel of its own: expr's leaf `value` stands for the reduced value and
    // every other leaf is a scalar (1-element) operand. The kernel that writes
    // the result (the finishing kernel of a split reduction) also writes
    // expr.root, converted to out_dtype, to out, at the same position.
    struct StoreEpilogue {
        Expr expr;
        int value = -1;
        void* out = nullptr;
        DType out_dtype = DType::Float32;
    };
    ReducePlan plan_reduce(const Expr& expr, const std::vector<int>& in_shape, const std::vector<int>& axes, ReduceOp op,
                           void* out, int compute_units, bool launch_only = false, const StoreEpilogue* epilogue = nullptr);
    // Generated kernels launched by this process so far (tests count fusions).
    unsigned long long kernel_launches();
    void bind_workspace(ReducePlan& plan, void* workspace);

    // Source text of a planned kernel: a plan that hit the kernel cache after
    // its kernel was compiled carries only the handle, and this returns the
    // text the cache kept (diagnostics and compile-only checks).
    std::string kernel_source(const KernelLaunch& k);
    // hipRTC options every generated kernel is compiled with.
    const std::vector<std::string>& rtc_options();
    // Compile (cached) and launch.
    void launch(const KernelLaunch& k);

}
