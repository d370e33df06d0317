// ormi_hip_reduce: the C-ABI reduction entry of the device layer.
//
// Replaces the reference's cuda::sum kernel entry
// (csrc/backend/cuda/kernels/reduce/cuda_sum.cuh:5-11, sum.cu:12-97) for callers
// that hold only this library: the input is a raw strided view, the output a
// contiguous buffer. The kernels are the fusion scheduler's own: this file runs
// the same code generator (backend/hip/codegen.cpp, built into this library
// with hidden symbols) on an expression that is just the input, then compiles
// through the library's hipRTC cache and launches on its stream.
//
// ormi_hip_reduce_map is the same reduction over a caller's element-wise tape
// (the ormi_hip_map descriptor) evaluated as the kernel's prologue, as the
// fusion scheduler fuses a reduction's producer.
//
// Built with -fvisibility=hidden: only the extern "C" functions are exported.
#include <algorithm>
#include <cstdint>
#include <exception>
#include <mutex>
#include <string>
#include <vector>

#include "backend/hip/kernel_gen.h"
#include "map_tape.h"
#include "ormi_hip_internal.h"

#define ORMI_EXPORT extern "C" __attribute__((visibility("default")))

namespace {
    using ormi::DType;
    using namespace ormi::hip;
    using ormi_hip::fail;

    struct Request {
        std::vector<int> shape, axes;  // axes sorted; every dim when the caller gave none
        ReduceOp op = ReduceOp::Sum;
        DType dtype = DType::Float32;
        long long in_numel = 1, out_numel = 1;
    };

    // op and axes over shape (the input's, or the prologue's): r->shape,
    // r->axes (sorted; every dim when naxes is 0), in_numel, out_numel.
    int check_reduction(const std::string& who, int op, int ndim, const int* shape, int naxes, const int* axes,
                        const void* out, Request* r) {
        switch (op) {
            case ORMI_REDUCE_SUM: r->op = ReduceOp::Sum; break;
            case ORMI_REDUCE_MAX: r->op = ReduceOp::Max; break;
            case ORMI_REDUCE_ARGMAX: r->op = ReduceOp::Argmax; break;
            default: return fail(ORMI_HIP_ERR_INVALID, who + ": op must be ORMI_REDUCE_SUM, _MAX or _ARGMAX");
        }
        if (ndim < 0 || ndim > ORMI_REDUCE_MAX_DIMS) return fail(ORMI_HIP_ERR_INVALID, who + ": ndim must be 0..8");
        if (naxes < 0 || naxes > ndim) return fail(ORMI_HIP_ERR_INVALID, who + ": naxes must be 0..ndim");
        r->shape.assign(shape, shape + ndim);
        r->in_numel = r->out_numel = 1;
        for (int e : r->shape) {
            if (e < 0) return fail(ORMI_HIP_ERR_INVALID, who + ": negative extent");
            if (e > 0 && r->in_numel > (1LL << 62) / e) return fail(ORMI_HIP_ERR_INVALID, who + ": more than 2^62 elements");
            r->in_numel *= e;
        }
        std::vector<bool> reduced(ndim, naxes == 0);
        for (int i = 0; i < naxes; ++i) {
            const int a = axes[i];
            if (a < 0 || a >= ndim) return fail(ORMI_HIP_ERR_INVALID, who + ": axis out of range");
            if (reduced[a]) return fail(ORMI_HIP_ERR_INVALID, who + ": repeated axis");
            reduced[a] = true;
        }
        r->axes.clear();
        for (int a = 0; a < ndim; ++a) {
            if (reduced[a]) r->axes.push_back(a);
            else r->out_numel *= r->shape[a];
        }
        if (r->out_numel > 0 && !out) return fail(ORMI_HIP_ERR_INVALID, who + ": null output");
        // fp32 values, or int64 indices for ARGMAX
        if ((uintptr_t)out % (r->op == ReduceOp::Argmax ? 8 : 4) != 0)
            return fail(ORMI_HIP_ERR_INVALID, who + ": output is not aligned to its element size");
        return ORMI_HIP_OK;
    }

    int check(const ormi_reduce_desc* d, Request* r) {
        if (!d) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: null descriptor");
        if (d->op != ORMI_REDUCE_SUM && d->op != ORMI_REDUCE_MAX && d->op != ORMI_REDUCE_ARGMAX)
            return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: op must be ORMI_REDUCE_SUM, _MAX or _ARGMAX");
        switch (d->in_dtype) {
            case ORMI_DTYPE_F32: r->dtype = DType::Float32; break;
            case ORMI_DTYPE_BF16: r->dtype = DType::BFloat16; break;
            case ORMI_DTYPE_F16: r->dtype = DType::Float16; break;
            case ORMI_DTYPE_I32: r->dtype = DType::Int32; break;
            case ORMI_DTYPE_I64: r->dtype = DType::Int64; break;
            case ORMI_DTYPE_BOOL: r->dtype = DType::Bool; break;
            default: return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: unknown input dtype");
        }
        const int rc = check_reduction("ormi_hip_reduce", d->op, d->ndim, d->shape, d->naxes, d->axes, d->out, r);
        if (rc != ORMI_HIP_OK) return rc;
        if (r->in_numel > 0 && !d->in) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: null input");
        if ((uintptr_t)d->in % ormi::dtype_size(r->dtype) != 0)
            return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: input is not aligned to its element size");
        return ORMI_HIP_OK;
    }

    Expr input_expr(const ormi_reduce_desc* d, const Request& r) {
        Expr e;
        Leaf L;
        L.ptr = d->in;
        L.dtype = r.dtype;
        L.st.assign(d->strides, d->strides + d->ndim);
        e.leaves.push_back(std::move(L));
        e.root = 0;
        e.roots = {0};
        return e;
    }

    // Library-owned partials buffer for callers that pass no workspace; the lock
    // is held until the kernels that use it are enqueued.
    std::mutex g_mu;
    void* g_ws = nullptr;
    size_t g_ws_bytes = 0;

    int own_workspace_locked(size_t bytes, void** out) {
        if (bytes > g_ws_bytes) {
            if (g_ws) {
                if (ormi_hip_synchronize() != ORMI_HIP_OK || ormi_hip_free(g_ws) != ORMI_HIP_OK)
                    return ORMI_HIP_ERR_RUNTIME;
                g_ws = nullptr;
                g_ws_bytes = 0;
            }
            const int rc = ormi_hip_malloc(&g_ws, bytes);
            if (rc != ORMI_HIP_OK) return rc;
            g_ws_bytes = bytes;
        }
        *out = g_ws;
        return ORMI_HIP_OK;
    }
}

namespace {
    // Workspace bytes of the reduction of expr (0 when it takes one pass).
    int workspace_of(const std::string& who, const Expr& expr, const Request& r, void* out, size_t* bytes) {
        *bytes = 0;
        if (r.out_numel == 0 || r.in_numel == 0) return ORMI_HIP_OK;
        const int rc = ormi_hip::ensure_init();
        if (rc != ORMI_HIP_OK) return rc;
        try {
            const ReducePlan plan = plan_reduce(expr, r.shape, r.axes, r.op, out, ormi_hip::compute_units());
            *bytes = plan.two_pass ? plan.workspace_bytes : 0;
        } catch (const std::exception& e) {
            return fail(ORMI_HIP_ERR_INVALID, who + "_workspace_size: " + e.what());
        }
        return ORMI_HIP_OK;
    }

    // Plan, bind a workspace (the caller's, else the library's) and launch.
    int run(const std::string& who, const Expr& expr, const Request& r, void* out, void* workspace,
            size_t workspace_bytes) {
        // the partials are fp32 values and int32 positions
        if ((uintptr_t)workspace % 4 != 0) return fail(ORMI_HIP_ERR_INVALID, who + ": workspace is not 4-byte aligned");
        if (r.out_numel == 0) return ORMI_HIP_OK;
        int rc = ormi_hip::ensure_init();
        if (rc != ORMI_HIP_OK) return rc;
        if (r.in_numel == 0) {
            if (r.op != ReduceOp::Sum)
                return fail(ORMI_HIP_ERR_INVALID, who + ": zero-size array to reduction operation maximum which has no identity");
            const float zero = 0.0f;
            return ormi_hip_fill(out, &zero, 4, (size_t)r.out_numel);
        }
        try {
            ReducePlan plan = plan_reduce(expr, r.shape, r.axes, r.op, out, ormi_hip::compute_units(), true);
            std::unique_lock<std::mutex> lock(g_mu, std::defer_lock);
            if (plan.two_pass) {
                void* ws = workspace;
                if (ws) {
                    if (workspace_bytes < plan.workspace_bytes)
                        return fail(ORMI_HIP_ERR_INVALID, who + ": workspace smaller than " + who + "_workspace_size() (" +
                                                              std::to_string(plan.workspace_bytes) + " bytes)");
                } else {
                    lock.lock();
                    rc = own_workspace_locked(plan.workspace_bytes, &ws);
                    if (rc != ORMI_HIP_OK) return rc;
                }
                bind_workspace(plan, ws);
            }
            launch(plan.first);
            if (plan.two_pass) launch(plan.second);
        } catch (const std::exception& e) {
            return fail(ORMI_HIP_ERR_RUNTIME, who + ": " + e.what());
        }
        return ORMI_HIP_OK;
    }

    // The fused form: the prologue's tape is the reduction's input expression.
    int check_map(const ormi_reduce_map_desc* d, ormi_hip::MapTape* t, Request* r) {
        if (!d) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce_map: null descriptor");
        if (d->op != ORMI_REDUCE_SUM && d->op != ORMI_REDUCE_MAX && d->op != ORMI_REDUCE_ARGMAX)
            return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce_map: op must be ORMI_REDUCE_SUM, _MAX or _ARGMAX");
        if (!d->prologue) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce_map: null prologue");
        int rc = ormi_hip::parse_map_tape(d->prologue, "ormi_hip_reduce_map", false, t);
        if (rc != ORMI_HIP_OK) return rc;
        return check_reduction("ormi_hip_reduce_map", d->op, d->prologue->ndim, d->prologue->shape, d->naxes, d->axes,
                               d->out, r);
    }
}

ORMI_EXPORT int ormi_hip_reduce_workspace_size(const ormi_reduce_desc* d, size_t* bytes) {
    if (!bytes) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce_workspace_size: null output");
    *bytes = 0;
    Request r;
    const int rc = check(d, &r);
    if (rc != ORMI_HIP_OK) return rc;
    return workspace_of("ormi_hip_reduce", input_expr(d, r), r, d->out, bytes);
}

ORMI_EXPORT int ormi_hip_reduce(const ormi_reduce_desc* d) {
    Request r;
    const int rc = check(d, &r);
    if (rc != ORMI_HIP_OK) return rc;
    return run("ormi_hip_reduce", input_expr(d, r), r, d->out, d->workspace, d->workspace_bytes);
}

ORMI_EXPORT int ormi_hip_reduce_map_workspace_size(const ormi_reduce_map_desc* d, size_t* bytes) {
    if (!bytes) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce_map_workspace_size: null output");
    *bytes = 0;
    ormi_hip::MapTape t;
    Request r;
    const int rc = check_map(d, &t, &r);
    if (rc != ORMI_HIP_OK) return rc;
    return workspace_of("ormi_hip_reduce_map", t.expr, r, d->out, bytes);
}

ORMI_EXPORT int ormi_hip_reduce_map(const ormi_reduce_map_desc* d) {
    ormi_hip::MapTape t;
    Request r;
    const int rc = check_map(d, &t, &r);
    if (rc != ORMI_HIP_OK) return rc;
    return run("ormi_hip_reduce_map", t.expr, r, d->out, d->workspace, d->workspace_bytes);
}
