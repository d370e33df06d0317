// ormi_hip_map: the C-ABI element-wise entry of the device layer.
//
// Replaces the reference's element-wise JIT (cuda::execute_jit,
// csrc/backend/cuda/jit.cu:13-44, over the tape of compiler.cu:22-51) for
// callers that hold only this library: they pass the tape (leaves with strides
// aligned to the map's shape, instructions over earlier values) and contiguous
// outputs. The kernel is the fusion scheduler's own: this file runs the same
// code generator (backend/hip/codegen.cpp, built into this library with hidden
// symbols) with the same built-in lowerings, so a tape gives the same kernel
// text on either path, then launches it through the library's queue.
//
// Built with -fvisibility=hidden: only the extern "C" function is exported.
#include <cstdint>
#include <exception>
#include <string>
#include <vector>

#include "backend/hip/kernel_gen.h"
#include "map_tape.h"
#include "ormi_hip_internal.h"

#define ORMI_EXPORT extern "C" __attribute__((visibility("default")))

namespace {
    using ormi::DType;
    using ormi::ops::OpEnum;
    using namespace ormi::hip;
    using ormi_hip::fail;

    bool to_dtype(int d, DType* out) {
        switch (d) {
            case ORMI_DTYPE_F32: *out = DType::Float32; return true;
            case ORMI_DTYPE_BF16: *out = DType::BFloat16; return true;
            case ORMI_DTYPE_F16: *out = DType::Float16; return true;
            case ORMI_DTYPE_I32: *out = DType::Int32; return true;
            case ORMI_DTYPE_I64: *out = DType::Int64; return true;
            case ORMI_DTYPE_BOOL: *out = DType::Bool; return true;
        }
        return false;
    }

    // ORMI_MAP_* -> the core's op (its arity comes from ops::op_arity).
    bool to_op(int op, OpEnum* out) {
        static const OpEnum table[] = {OpEnum::NEG,  OpEnum::EXP,       OpEnum::LOG,     OpEnum::SIN,
                                       OpEnum::COS,  OpEnum::ADD,       OpEnum::SUB,     OpEnum::MUL,
                                       OpEnum::DIV,  OpEnum::POW,       OpEnum::RELU,    OpEnum::STEP,
                                       OpEnum::TANH, OpEnum::TANH_GRAD, OpEnum::SIGMOID, OpEnum::SIGMOID_GRAD,
                                       OpEnum::GELU, OpEnum::GELU_GRAD, OpEnum::EQ,      OpEnum::CAST};
        if (op < 0 || op >= (int)(sizeof(table) / sizeof(table[0]))) return false;
        *out = table[op];
        return true;
    }

}  // namespace

namespace ormi_hip {
    using ormi::DType;
    using ormi::ops::OpEnum;
    using ormi::hip::Expr;
    using ormi::hip::Inst;
    using ormi::hip::Leaf;
    using ormi::hip::builtin_lowering;

    int parse_map_tape(const ormi_map_desc* d, const char* who_c, bool with_buffers, MapTape* t) {
        const std::string who(who_c);
        if (!d) return fail(ORMI_HIP_ERR_INVALID, who + ": null descriptor");
        if (d->ndim < 0 || d->ndim > ORMI_MAP_MAX_DIMS) return fail(ORMI_HIP_ERR_INVALID, who + ": ndim must be 0..8");
        t->shape.assign(d->shape, d->shape + d->ndim);
        for (int e : t->shape) {
            if (e < 0) return fail(ORMI_HIP_ERR_INVALID, who + ": negative extent");
            if (e > 0 && t->numel > (1LL << 62) / e) return fail(ORMI_HIP_ERR_INVALID, who + ": more than 2^62 elements");
            t->numel *= e;
        }
        if (d->num_leaves < 0 || (d->num_leaves > 0 && !d->leaves))
            return fail(ORMI_HIP_ERR_INVALID, who + ": num_leaves must be >= 0, with a leaves array");
        if (d->num_insts < 0 || (d->num_insts > 0 && !d->insts))
            return fail(ORMI_HIP_ERR_INVALID, who + ": num_insts must be >= 0, with an insts array");
        if (with_buffers) {
            if (d->num_outputs < 1 || d->num_outputs > ORMI_MAP_MAX_OUTPUTS || !d->output_values || !d->outputs ||
                !d->output_dtypes)
                return fail(ORMI_HIP_ERR_INVALID, who + ": num_outputs must be 1..16, with values, buffers and dtypes");
        } else if (d->num_outputs != 1 || !d->output_values) {
            return fail(ORMI_HIP_ERR_INVALID, who + ": the prologue has exactly one output value (num_outputs = 1)");
        }
        const int nval = d->num_leaves + d->num_insts;
        Expr& e = t->expr;
        for (int i = 0; i < d->num_leaves; ++i) {
            const ormi_map_leaf& s = d->leaves[i];
            Leaf L;
            if (!to_dtype(s.dtype, &L.dtype)) return fail(ORMI_HIP_ERR_INVALID, who + ": leaf " + std::to_string(i) + " has an unknown dtype");
            if (!s.ptr && t->numel > 0) return fail(ORMI_HIP_ERR_INVALID, who + ": leaf " + std::to_string(i) + " is null");
            if ((uintptr_t)s.ptr % ormi::dtype_size(L.dtype) != 0)
                return fail(ORMI_HIP_ERR_INVALID, who + ": leaf " + std::to_string(i) + " is not aligned to its element size");
            L.ptr = s.ptr;
            L.scalar = s.scalar != 0;
            L.st.assign(d->ndim, 0);
            if (!L.scalar)
                for (int k = 0; k < d->ndim; ++k) L.st[k] = d->shape[k] == 1 ? 0 : s.strides[k];
            e.leaves.push_back(std::move(L));
        }
        for (int k = 0; k < d->num_insts; ++k) {
            const ormi_map_inst& s = d->insts[k];
            const std::string where = who + ": instruction " + std::to_string(k);
            Inst in;
            if (!to_op(s.op, &in.op)) return fail(ORMI_HIP_ERR_INVALID, where + " has an unknown op");
            const int self = d->num_leaves + k;
            if (s.a < 0 || s.a >= self) return fail(ORMI_HIP_ERR_INVALID, where + ": operand a must be an earlier value");
            in.a = s.a;
            if (ormi::ops::op_arity(in.op) == 2) {
                if (s.b < 0 || s.b >= self) return fail(ORMI_HIP_ERR_INVALID, where + ": operand b must be an earlier value");
                in.b = s.b;
            }
            if (in.op == OpEnum::CAST) {
                if (!to_dtype(s.dtype, &in.cast) ||
                    (in.cast != DType::Float32 && in.cast != DType::BFloat16 && in.cast != DType::Float16))
                    return fail(ORMI_HIP_ERR_INVALID, where + ": CAST rounds to bf16, f16 or f32 only");
            } else {
                in.lower = builtin_lowering(in.op);
            }
            e.insts.push_back(in);
        }
        for (int o = 0; o < d->num_outputs; ++o) {
            const int v = d->output_values[o];
            if (v < 0 || v >= nval) return fail(ORMI_HIP_ERR_INVALID, who + ": output " + std::to_string(o) + " names no value");
            e.roots.push_back(v);
            if (!with_buffers) continue;
            DType dt;
            if (!to_dtype(d->output_dtypes[o], &dt)) return fail(ORMI_HIP_ERR_INVALID, who + ": output " + std::to_string(o) + " has an unknown dtype");
            if (!d->outputs[o] && t->numel > 0) return fail(ORMI_HIP_ERR_INVALID, who + ": output " + std::to_string(o) + " is null");
            if ((uintptr_t)d->outputs[o] % ormi::dtype_size(dt) != 0)
                return fail(ORMI_HIP_ERR_INVALID, who + ": output " + std::to_string(o) + " is not aligned to its element size");
            t->outs.push_back(d->outputs[o]);
            t->out_dtypes.push_back(dt);
        }
        e.root = e.roots[0];
        return ORMI_HIP_OK;
    }
}

ORMI_EXPORT int ormi_hip_map(const ormi_map_desc* d) {
    ormi_hip::MapTape r;
    int rc = ormi_hip::parse_map_tape(d, "ormi_hip_map", true, &r);
    if (rc != ORMI_HIP_OK) return rc;
    if (r.numel == 0) return ORMI_HIP_OK;
    rc = ormi_hip::ensure_init();
    if (rc != ORMI_HIP_OK) return rc;
    try {
        launch(plan_map_multi(r.expr, r.shape, r.outs, r.out_dtypes, ormi_hip::compute_units(), true));
    } catch (const std::exception& e) {
        return fail(ORMI_HIP_ERR_RUNTIME, std::string("ormi_hip_map: ") + e.what());
    }
    return ORMI_HIP_OK;
}
