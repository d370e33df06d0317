// SUM (reference: csrc/core/ops/reduce/sum.cpp:11-100) plus the additive MAX
// and ARGMAX reductions, which share its shape rule.
#include <stdexcept>
#include <algorithm>
#include "core/ops/api.h"
#include "core/shape.h"
#include "core/adjoint.h"
#include "core/registry.h"

namespace ormi {
    using ops::OpEnum;
    using NodeVec = std::vector<std::shared_ptr<Node>>;

    static std::vector<int> normalize_axes(const std::vector<int>& axes, int ndim) {
        std::vector<int> out;
        for (int a : axes) {
            int ax = a < 0 ? a + ndim : a;
            if (ax < 0 || ax >= ndim) throw std::runtime_error("Reduction axis out of range.");
            if (std::find(out.begin(), out.end(), ax) == out.end()) out.push_back(ax);
        }
        std::sort(out.begin(), out.end());
        return out;
    }

    static std::shared_ptr<Node> make_reduce(OpEnum op, ops::NodePtr x, const std::vector<int>& axes, bool keepdims) {
        if (!x) throw std::runtime_error("Reduction got a null operand.");
        ReduceAttrs attrs;
        attrs.axes = normalize_axes(axes, (int)x->view.shape.size());
        attrs.keepdims = keepdims;
        return std::make_shared<Node>(op, NodeVec{x}, x->device, attrs);
    }

    namespace ops {
        NodePtr sum(NodePtr x, const std::vector<int>& axes, bool keepdims) { return make_reduce(OpEnum::SUM, x, axes, keepdims); }
        NodePtr max(NodePtr x, const std::vector<int>& axes, bool keepdims) { return make_reduce(OpEnum::MAX, x, axes, keepdims); }
        NodePtr argmax(NodePtr x, const std::vector<int>& axes, bool keepdims) {
            if (axes.size() > 1) throw std::runtime_error("ARGMAX takes one axis (or none for the flattened tensor).");
            return make_reduce(OpEnum::ARGMAX, x, axes, keepdims);
        }
    }

    // Output shape: reduced axes dropped (or kept as 1 with keepdims); no axes
    // means every axis (reference: csrc/core/ops/reduce/sum.cpp:25-55).
    static std::vector<int> infer_reduce_shape(const NodeVec& parents, const OpAttributes& attrs) {
        if (parents.empty()) throw std::runtime_error("Reduction requires 1 parent.");
        const auto& in = parents[0]->view.shape;
        const auto& r = std::get<ReduceAttrs>(attrs);
        std::vector<int> out;
        if (r.axes.empty()) {
            if (r.keepdims) out.assign(in.size(), 1);
            return out;
        }
        for (size_t d = 0; d < in.size(); ++d) {
            const bool reduced = std::find(r.axes.begin(), r.axes.end(), (int)d) != r.axes.end();
            if (!reduced) out.push_back(in[d]);
            else if (r.keepdims) out.push_back(1);
        }
        return out;
    }

    // Re-insert the reduced axes of a reduction result (as 1s) and broadcast it
    // back over x's shape: RESHAPE then EXPAND, both zero-copy views.
    static std::shared_ptr<Node> expand_to_input(const std::shared_ptr<Node>& reduced, const std::shared_ptr<Node>& x,
                                                 const ReduceAttrs& r, const Device& dev) {
        std::shared_ptr<Node> e = reduced;
        if (!r.keepdims) {
            std::vector<int> target = x->view.shape;
            if (r.axes.empty()) std::fill(target.begin(), target.end(), 1);
            else for (int ax : r.axes) target[ax] = 1;
            e = std::make_shared<Node>(OpEnum::RESHAPE, NodeVec{e}, dev, ReshapeAttrs{target});
        }
        return std::make_shared<Node>(OpEnum::EXPAND, NodeVec{e}, dev, ExpandAttrs{x->view.shape});
    }

    static void adjoint_sum(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (!x->requires_grad) return;
        const auto& r = std::get<ReduceAttrs>(n->attrs);
        accumulate_grad(x, expand_to_input(n->grad, x, r, n->device), n->device);
    }

    // d max = dZ routed to every position equal to the maximum.
    static void adjoint_max(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (!x->requires_grad) return;
        const auto& r = std::get<ReduceAttrs>(n->attrs);
        auto dz = expand_to_input(n->grad, x, r, n->device);
        auto m = expand_to_input(n, x, r, n->device);
        auto mask = std::make_shared<Node>(OpEnum::EQ, NodeVec{x, m}, n->device);
        accumulate_grad(x, std::make_shared<Node>(OpEnum::MUL, NodeVec{dz, mask}, n->device), n->device);
    }

    static RegisterShape rs_sum(OpEnum::SUM, infer_reduce_shape);
    static RegisterShape rs_max(OpEnum::MAX, infer_reduce_shape);
    static RegisterShape rs_argmax(OpEnum::ARGMAX, infer_reduce_shape);
    static RegisterAdjoint ra_sum(OpEnum::SUM, adjoint_sum);
    static RegisterAdjoint ra_max(OpEnum::MAX, adjoint_max);
}
