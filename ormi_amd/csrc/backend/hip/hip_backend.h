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
#include "backend/hip/kernel_gen.h"

namespace ormi::hip {
    using NodePtr = std::shared_ptr<Node>;

    // OpEnum -> HIP C expression over operand expressions.
    class HIPLoweringRegistry {
    public:
        static void register_func(ops::OpEnum op, LoweringFunc f);
        static LoweringFunc get(ops::OpEnum op);  // throws when op has no lowering
        static bool has(ops::OpEnum op);
        // The registered function (stable for the process), or nullptr.
        static const LoweringFunc* find(ops::OpEnum op);
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
    // The unrealized SUM or MAX whose store epilogue the element-wise region of
    // n can be (n's region reads only it and realized scalars, and it has n's
    // shape), else nullptr. The scheduler then realizes both with one kernel.
    NodePtr epilogue_reduction(const NodePtr& n);

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
    // Pairs of products the scheduler launched as one grouped GEMM
    // (ormi_hip_gemm_pair) so far.
    uint64_t gemm_pair_count();

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
