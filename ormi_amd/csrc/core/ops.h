#pragma once

namespace ormi::ops {
    // The values up to FRAC_DERIV are the reference's op set in the reference's
    // order (csrc/core/ops.h:4-10). The rest are the ops the benchmark configs
    // need and the reference lacks: activations with their derivative ops
    // (adjoints build these instead of allocating constants), MAX/ARGMAX
    // reductions, an equality mask for the MAX adjoint, and a dtype CAST.
    enum class OpEnum {
        LEAF, CONST,
        NEG, EXP, LOG, SIN, COS,
        ADD, SUB, MUL, DIV, POW, MATMUL,
        SUM, TRANSPOSE, RESHAPE, EXPAND,
        FRAC_DERIV,
        RELU, STEP, TANH, TANH_GRAD, SIGMOID, SIGMOID_GRAD, GELU, GELU_GRAD,
        MAX, ARGMAX, EQ, CAST
    };

    const char* op_name(OpEnum op);
    bool is_pointwise(OpEnum op);   // element-wise ops a fused kernel may contain
    bool is_reduction(OpEnum op);   // SUM, MAX, ARGMAX
    int op_arity(OpEnum op);        // 1 or 2 for pointwise ops, 0 otherwise
}
