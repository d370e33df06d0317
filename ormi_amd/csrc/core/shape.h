#pragma once
#include <vector>
#include <memory>
#include "core/ops.h"
#include "core/attributes.h"
#include "core/registry.h"

namespace ormi {
    struct Node;

    // Shape and element strides of a node. Strides of 0 mark broadcast axes.
    struct TensorView {
        std::vector<int> shape;
        std::vector<int> strides;
        bool is_contiguous() const;
    };

    // v as an int, or a std::runtime_error naming `what` when it does not fit.
    int checked_extent(long long v, const char* what);
    std::vector<int> calc_contiguous_strides(const std::vector<int>& shape);
    std::vector<int> broadcast_shapes(const std::vector<int>& a, const std::vector<int>& b);
    std::vector<int> infer_shape(ops::OpEnum op, const std::vector<std::shared_ptr<Node>>& parents, const OpAttributes& attrs);
    std::vector<int> infer_unary_shape(const std::vector<std::shared_ptr<Node>>& parents, const OpAttributes&);
    std::vector<int> infer_binary_shape(const std::vector<std::shared_ptr<Node>>& parents, const OpAttributes&);
    long long shape_numel(const std::vector<int>& shape);
}
