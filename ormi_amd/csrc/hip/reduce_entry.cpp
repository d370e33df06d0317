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
// Built with -fvisibility=hidden: only the two extern "C" functions are exported.
#include <algorithm>
#include <exception>
#include <mutex>
#include <string>
#include <vector>

#include "backend/hip/kernel_gen.h"
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

    int check(const ormi_reduce_desc* d, Request* r) {
        if (!d) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: null descriptor");
        switch (d->op) {
            case ORMI_REDUCE_SUM: r->op = ReduceOp::Sum; break;
            case ORMI_REDUCE_MAX: r->op = ReduceOp::Max; break;
            case ORMI_REDUCE_ARGMAX: r->op = ReduceOp::Argmax; break;
            default: return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: op must be ORMI_REDUCE_SUM, _MAX or _ARGMAX");
        }
        switch (d->in_dtype) {
            case ORMI_DTYPE_F32: r->dtype = DType::Float32; break;
            case ORMI_DTYPE_BF16: r->dtype = DType::BFloat16; break;
            case ORMI_DTYPE_F16: r->dtype = DType::Float16; break;
            case ORMI_DTYPE_I32: r->dtype = DType::Int32; break;
            case ORMI_DTYPE_I64: r->dtype = DType::Int64; break;
            case ORMI_DTYPE_BOOL: r->dtype = DType::Bool; break;
            default: return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: unknown input dtype");
        }
        if (d->ndim < 0 || d->ndim > ORMI_REDUCE_MAX_DIMS)
            return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: ndim must be 0..8");
        if (d->naxes < 0 || d->naxes > d->ndim) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: naxes must be 0..ndim");
        r->shape.assign(d->shape, d->shape + d->ndim);
        for (int e : r->shape) {
            if (e < 0) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: negative extent");
            if (e > 0 && r->in_numel > (1LL << 62) / e) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: more than 2^62 elements");
            r->in_numel *= e;
        }
        std::vector<bool> reduced(d->ndim, d->naxes == 0);
        for (int i = 0; i < d->naxes; ++i) {
            const int a = d->axes[i];
            if (a < 0 || a >= d->ndim) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: axis out of range");
            if (reduced[a]) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: repeated axis");
            reduced[a] = true;
        }
        r->axes.clear();
        for (int a = 0; a < d->ndim; ++a) {
            if (reduced[a]) r->axes.push_back(a);
            else r->out_numel *= r->shape[a];
        }
        if (r->out_numel > 0 && !d->out) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: null output");
        if (r->in_numel > 0 && !d->in) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: null input");
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

ORMI_EXPORT int ormi_hip_reduce_workspace_size(const ormi_reduce_desc* d, size_t* bytes) {
    if (!bytes) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce_workspace_size: null output");
    *bytes = 0;
    Request r;
    int rc = check(d, &r);
    if (rc != ORMI_HIP_OK) return rc;
    if (r.out_numel == 0 || r.in_numel == 0) return ORMI_HIP_OK;
    rc = ormi_hip::ensure_init();
    if (rc != ORMI_HIP_OK) return rc;
    try {
        const ReducePlan plan = plan_reduce(input_expr(d, r), r.shape, r.axes, r.op, d->out, ormi_hip::compute_units());
        *bytes = plan.two_pass ? plan.workspace_bytes : 0;
    } catch (const std::exception& e) {
        return fail(ORMI_HIP_ERR_INVALID, std::string("ormi_hip_reduce_workspace_size: ") + e.what());
    }
    return ORMI_HIP_OK;
}

ORMI_EXPORT int ormi_hip_reduce(const ormi_reduce_desc* d) {
    Request r;
    int rc = check(d, &r);
    if (rc != ORMI_HIP_OK) return rc;
    if (r.out_numel == 0) return ORMI_HIP_OK;
    rc = ormi_hip::ensure_init();
    if (rc != ORMI_HIP_OK) return rc;
    if (r.in_numel == 0) {
        if (r.op != ReduceOp::Sum)
            return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: zero-size array to reduction operation maximum which has no identity");
        const float zero = 0.0f;
        return ormi_hip_fill(d->out, &zero, 4, (size_t)r.out_numel);
    }
    try {
        ReducePlan plan = plan_reduce(input_expr(d, r), r.shape, r.axes, r.op, d->out, ormi_hip::compute_units(), true);
        std::unique_lock<std::mutex> lock(g_mu, std::defer_lock);
        if (plan.two_pass) {
            void* ws = d->workspace;
            if (ws) {
                if (d->workspace_bytes < plan.workspace_bytes)
                    return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_reduce: workspace smaller than ormi_hip_reduce_workspace_size() (" +
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
        return fail(ORMI_HIP_ERR_RUNTIME, std::string("ormi_hip_reduce: ") + e.what());
    }
    return ORMI_HIP_OK;
}
