// Element-wise ops: constructors, shape rules and adjoints.
// Reference rules followed: csrc/core/ops/pointwise/{add,sub,mul,div,pow,neg,exp,log,sin,cos}.cpp.
// RELU/TANH/SIGMOID/GELU/EQ are additive; their adjoints use derivative ops
// (STEP, TANH_GRAD, SIGMOID_GRAD, GELU_GRAD) so no constant buffer is allocated
// while the backward graph is built.
#include <stdexcept>
#include "core/ops/api.h"
#include "core/shape.h"
#include "core/adjoint.h"
#include "core/registry.h"

namespace ormi {
    using ops::OpEnum;
    using NodeVec = std::vector<std::shared_ptr<Node>>;

    namespace ops {
        NodePtr binary(OpEnum op, NodePtr a, NodePtr b) {
            if (!a || !b) throw std::runtime_error("Pointwise op got a null operand.");
            return std::make_shared<Node>(op, NodeVec{a, b}, a->device);
        }
        NodePtr unary(OpEnum op, NodePtr a) {
            if (!a) throw std::runtime_error("Pointwise op got a null operand.");
            return std::make_shared<Node>(op, NodeVec{a}, a->device);
        }
        NodePtr add(NodePtr a, NodePtr b) { return binary(OpEnum::ADD, a, b); }
        NodePtr sub(NodePtr a, NodePtr b) { return binary(OpEnum::SUB, a, b); }
        NodePtr mul(NodePtr a, NodePtr b) { return binary(OpEnum::MUL, a, b); }
        NodePtr div(NodePtr a, NodePtr b) { return binary(OpEnum::DIV, a, b); }
        NodePtr pow(NodePtr a, NodePtr b) { return binary(OpEnum::POW, a, b); }
        NodePtr eq(NodePtr a, NodePtr b) { return binary(OpEnum::EQ, a, b); }
        NodePtr neg(NodePtr a) { return unary(OpEnum::NEG, a); }
        NodePtr exp(NodePtr a) { return unary(OpEnum::EXP, a); }
        NodePtr log(NodePtr a) { return unary(OpEnum::LOG, a); }
        NodePtr sin(NodePtr a) { return unary(OpEnum::SIN, a); }
        NodePtr cos(NodePtr a) { return unary(OpEnum::COS, a); }
        NodePtr relu(NodePtr a) { return unary(OpEnum::RELU, a); }
        NodePtr step(NodePtr a) { return unary(OpEnum::STEP, a); }
        NodePtr tanh(NodePtr a) { return unary(OpEnum::TANH, a); }
        NodePtr sigmoid(NodePtr a) { return unary(OpEnum::SIGMOID, a); }
        NodePtr gelu(NodePtr a) { return unary(OpEnum::GELU, a); }
    }

    static std::shared_ptr<Node> mk(OpEnum op, NodeVec parents, const Device& dev) {
        return std::make_shared<Node>(op, std::move(parents), dev);
    }

    // Push a local gradient g into x after summing away broadcast axes.
    static void push(const std::shared_ptr<Node>& node, const std::shared_ptr<Node>& x, const std::shared_ptr<Node>& g) {
        accumulate_grad(x, unbroadcast(g, x->view.shape), node->device);
    }

    static void adjoint_add(std::shared_ptr<Node> n) {
        for (int i = 0; i < 2; ++i)
            if (n->parents[i]->requires_grad) push(n, n->parents[i], n->grad);
    }

    static void adjoint_sub(std::shared_ptr<Node> n) {
        auto x = n->parents[0], y = n->parents[1];
        if (x->requires_grad) push(n, x, n->grad);
        if (y->requires_grad) push(n, y, mk(OpEnum::NEG, {n->grad}, n->device));
    }

    static void adjoint_mul(std::shared_ptr<Node> n) {
        auto x = n->parents[0], y = n->parents[1];
        if (x->requires_grad) push(n, x, mk(OpEnum::MUL, {n->grad, y}, n->device));
        if (y->requires_grad) push(n, y, mk(OpEnum::MUL, {n->grad, x}, n->device));
    }

    static void adjoint_div(std::shared_ptr<Node> n) {
        auto x = n->parents[0], y = n->parents[1];
        if (x->requires_grad) push(n, x, mk(OpEnum::DIV, {n->grad, y}, n->device));
        if (y->requires_grad) {
            auto y2 = mk(OpEnum::MUL, {y, y}, n->device);
            auto q = mk(OpEnum::DIV, {x, y2}, n->device);
            push(n, y, mk(OpEnum::NEG, {mk(OpEnum::MUL, {n->grad, q}, n->device)}, n->device));
        }
    }

    // dX = dZ * y * x^(y-1); dY = dZ * x^y * ln(x) (reference: csrc/core/ops/pointwise/pow.cpp:14-43,
    // which also builds its `ones` operand as an eager buffer).
    static void adjoint_pow(std::shared_ptr<Node> n) {
        auto x = n->parents[0], y = n->parents[1];
        if (x->requires_grad) {
            auto one = std::make_shared<Node>(full(y->view.shape, 1.0f, y->device.type), false, y->device);
            auto ym1 = mk(OpEnum::SUB, {y, one}, n->device);
            auto xp = mk(OpEnum::POW, {x, ym1}, n->device);
            push(n, x, mk(OpEnum::MUL, {n->grad, mk(OpEnum::MUL, {y, xp}, n->device)}, n->device));
        }
        if (y->requires_grad) {
            auto lx = mk(OpEnum::LOG, {x}, n->device);
            push(n, y, mk(OpEnum::MUL, {n->grad, mk(OpEnum::MUL, {n, lx}, n->device)}, n->device));
        }
    }

    static void adjoint_neg(std::shared_ptr<Node> n) {
        if (n->parents[0]->requires_grad) push(n, n->parents[0], mk(OpEnum::NEG, {n->grad}, n->device));
    }
    static void adjoint_exp(std::shared_ptr<Node> n) {
        if (n->parents[0]->requires_grad) push(n, n->parents[0], mk(OpEnum::MUL, {n, n->grad}, n->device));
    }
    static void adjoint_log(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (x->requires_grad) push(n, x, mk(OpEnum::DIV, {n->grad, x}, n->device));
    }
    static void adjoint_sin(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (x->requires_grad) push(n, x, mk(OpEnum::MUL, {mk(OpEnum::COS, {x}, n->device), n->grad}, n->device));
    }
    static void adjoint_cos(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (x->requires_grad) {
            auto ns = mk(OpEnum::NEG, {mk(OpEnum::SIN, {x}, n->device)}, n->device);
            push(n, x, mk(OpEnum::MUL, {ns, n->grad}, n->device));
        }
    }
    // d relu(x) = dZ * [x > 0]
    static void adjoint_relu(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (x->requires_grad) push(n, x, mk(OpEnum::MUL, {n->grad, mk(OpEnum::STEP, {x}, n->device)}, n->device));
    }
    // d tanh(x) = dZ * (1 - y^2), y = tanh(x)
    static void adjoint_tanh(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (x->requires_grad) push(n, x, mk(OpEnum::MUL, {n->grad, mk(OpEnum::TANH_GRAD, {n}, n->device)}, n->device));
    }
    // d sigmoid(x) = dZ * y * (1 - y), y = sigmoid(x)
    static void adjoint_sigmoid(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (x->requires_grad) push(n, x, mk(OpEnum::MUL, {n->grad, mk(OpEnum::SIGMOID_GRAD, {n}, n->device)}, n->device));
    }
    // d gelu(x) = dZ * (Phi(x) + x * phi(x))
    static void adjoint_gelu(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (x->requires_grad) push(n, x, mk(OpEnum::MUL, {n->grad, mk(OpEnum::GELU_GRAD, {x}, n->device)}, n->device));
    }

    static RegisterShape rs_add(OpEnum::ADD, infer_binary_shape);
    static RegisterShape rs_sub(OpEnum::SUB, infer_binary_shape);
    static RegisterShape rs_mul(OpEnum::MUL, infer_binary_shape);
    static RegisterShape rs_div(OpEnum::DIV, infer_binary_shape);
    static RegisterShape rs_pow(OpEnum::POW, infer_binary_shape);
    static RegisterShape rs_eq(OpEnum::EQ, infer_binary_shape);
    static RegisterShape rs_neg(OpEnum::NEG, infer_unary_shape);
    static RegisterShape rs_exp(OpEnum::EXP, infer_unary_shape);
    static RegisterShape rs_log(OpEnum::LOG, infer_unary_shape);
    static RegisterShape rs_sin(OpEnum::SIN, infer_unary_shape);
    static RegisterShape rs_cos(OpEnum::COS, infer_unary_shape);
    static RegisterShape rs_relu(OpEnum::RELU, infer_unary_shape);
    static RegisterShape rs_step(OpEnum::STEP, infer_unary_shape);
    static RegisterShape rs_tanh(OpEnum::TANH, infer_unary_shape);
    static RegisterShape rs_tanhg(OpEnum::TANH_GRAD, infer_unary_shape);
    static RegisterShape rs_sig(OpEnum::SIGMOID, infer_unary_shape);
    static RegisterShape rs_sigg(OpEnum::SIGMOID_GRAD, infer_unary_shape);
    static RegisterShape rs_gelu(OpEnum::GELU, infer_unary_shape);
    static RegisterShape rs_gelug(OpEnum::GELU_GRAD, infer_unary_shape);

    static RegisterAdjoint ra_add(OpEnum::ADD, adjoint_add);
    static RegisterAdjoint ra_sub(OpEnum::SUB, adjoint_sub);
    static RegisterAdjoint ra_mul(OpEnum::MUL, adjoint_mul);
    static RegisterAdjoint ra_div(OpEnum::DIV, adjoint_div);
    static RegisterAdjoint ra_pow(OpEnum::POW, adjoint_pow);
    static RegisterAdjoint ra_neg(OpEnum::NEG, adjoint_neg);
    static RegisterAdjoint ra_exp(OpEnum::EXP, adjoint_exp);
    static RegisterAdjoint ra_log(OpEnum::LOG, adjoint_log);
    static RegisterAdjoint ra_sin(OpEnum::SIN, adjoint_sin);
    static RegisterAdjoint ra_cos(OpEnum::COS, adjoint_cos);
    static RegisterAdjoint ra_relu(OpEnum::RELU, adjoint_relu);
    static RegisterAdjoint ra_tanh(OpEnum::TANH, adjoint_tanh);
    static RegisterAdjoint ra_sig(OpEnum::SIGMOID, adjoint_sigmoid);
    static RegisterAdjoint ra_gelu(OpEnum::GELU, adjoint_gelu);
}
