#include <stdexcept>
#include "core/node.h"
#include "core/registry.h"
#include "runtime/runtime.h"

namespace ormi {
    // Leaf constructor (reference: csrc/core/node.cpp:8-13).
    Node::Node(std::shared_ptr<Buffer> mem, bool req_grad, Device dev)
        : op(ops::OpEnum::LEAF), data(std::move(mem)), requires_grad(req_grad), device(dev) {
        if (!data) throw std::runtime_error("Leaf node requires a buffer.");
        view.shape = data->shape;
        view.strides = calc_contiguous_strides(data->shape);
        dtype = data->dtype;
    }

    static DType result_dtype(ops::OpEnum op, const std::vector<std::shared_ptr<Node>>& parents, const OpAttributes& attrs) {
        switch (op) {
            case ops::OpEnum::TRANSPOSE: case ops::OpEnum::RESHAPE: case ops::OpEnum::EXPAND:
                return parents.empty() ? DType::Float32 : parents[0]->dtype;
            case ops::OpEnum::CAST: return std::get<CastAttrs>(attrs).dtype;
            case ops::OpEnum::ARGMAX: return DType::Int64;
            default: return DType::Float32;
        }
    }

    // Internal constructor (reference: csrc/core/node.cpp:16-32).
    Node::Node(ops::OpEnum operation, std::vector<std::shared_ptr<Node>> parent_nodes, Device dev, OpAttributes attributes)
        : op(operation), parents(std::move(parent_nodes)), requires_grad(false), device(dev), attrs(std::move(attributes)) {
        for (const auto& p : parents) {
            if (!p) throw std::runtime_error("Node parent is null.");
            if (p->requires_grad) requires_grad = true;
        }
        // Piecewise-constant and integer-valued results carry no gradient.
        if (op == ops::OpEnum::ARGMAX || op == ops::OpEnum::STEP || op == ops::OpEnum::EQ) requires_grad = false;

        view.shape = infer_shape(op, parents, attrs);
        const StrideInferFunc* stride_func = Registry<StrideInferFunc>::find(op);
        view.strides = stride_func ? (*stride_func)(parents, attrs, view.shape) : calc_contiguous_strides(view.shape);
        dtype = result_dtype(op, parents, attrs);
    }

    bool Node::is_realized() const { return data != nullptr; }

    void Node::realize() {
        if (!is_realized()) execute_graph(shared_from_this());
    }
}
