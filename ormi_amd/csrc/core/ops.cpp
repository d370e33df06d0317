#include "core/ops.h"

namespace ormi::ops {
    const char* op_name(OpEnum op) {
        switch (op) {
            case OpEnum::LEAF: return "LEAF"; case OpEnum::CONST: return "CONST";
            case OpEnum::NEG: return "NEG"; case OpEnum::EXP: return "EXP"; case OpEnum::LOG: return "LOG";
            case OpEnum::SIN: return "SIN"; case OpEnum::COS: return "COS";
            case OpEnum::ADD: return "ADD"; case OpEnum::SUB: return "SUB"; case OpEnum::MUL: return "MUL";
            case OpEnum::DIV: return "DIV"; case OpEnum::POW: return "POW"; case OpEnum::MATMUL: return "MATMUL";
            case OpEnum::SUM: return "SUM"; case OpEnum::TRANSPOSE: return "TRANSPOSE";
            case OpEnum::RESHAPE: return "RESHAPE"; case OpEnum::EXPAND: return "EXPAND";
            case OpEnum::FRAC_DERIV: return "FRAC_DERIV";
            case OpEnum::RELU: return "RELU"; case OpEnum::STEP: return "STEP";
            case OpEnum::TANH: return "TANH"; case OpEnum::TANH_GRAD: return "TANH_GRAD";
            case OpEnum::SIGMOID: return "SIGMOID"; case OpEnum::SIGMOID_GRAD: return "SIGMOID_GRAD";
            case OpEnum::GELU: return "GELU"; case OpEnum::GELU_GRAD: return "GELU_GRAD";
            case OpEnum::MAX: return "MAX"; case OpEnum::ARGMAX: return "ARGMAX";
            case OpEnum::EQ: return "EQ"; case OpEnum::CAST: return "CAST";
        }
        return "?";
    }

    int op_arity(OpEnum op) {
        switch (op) {
            case OpEnum::NEG: case OpEnum::EXP: case OpEnum::LOG: case OpEnum::SIN: case OpEnum::COS:
            case OpEnum::RELU: case OpEnum::STEP: case OpEnum::TANH: case OpEnum::TANH_GRAD:
            case OpEnum::SIGMOID: case OpEnum::SIGMOID_GRAD: case OpEnum::GELU: case OpEnum::GELU_GRAD:
            case OpEnum::CAST:
                return 1;
            case OpEnum::ADD: case OpEnum::SUB: case OpEnum::MUL: case OpEnum::DIV: case OpEnum::POW:
            case OpEnum::EQ:
                return 2;
            default:
                return 0;
        }
    }

    bool is_pointwise(OpEnum op) { return op_arity(op) > 0; }

    bool is_reduction(OpEnum op) {
        return op == OpEnum::SUM || op == OpEnum::MAX || op == OpEnum::ARGMAX;
    }
}
