#pragma once
#include <memory>
#include <vector>
#include "core/node.h"

// Op constructors. Each builds one lazy Node; nothing is computed here.
namespace ormi::ops {
    using NodePtr = std::shared_ptr<Node>;

    NodePtr add(NodePtr a, NodePtr b);
    NodePtr sub(NodePtr a, NodePtr b);
    NodePtr mul(NodePtr a, NodePtr b);
    NodePtr div(NodePtr a, NodePtr b);
    NodePtr pow(NodePtr a, NodePtr b);
    NodePtr eq(NodePtr a, NodePtr b);
    NodePtr neg(NodePtr a);
    NodePtr exp(NodePtr a);
    NodePtr log(NodePtr a);
    NodePtr sin(NodePtr a);
    NodePtr cos(NodePtr a);
    NodePtr relu(NodePtr a);
    NodePtr step(NodePtr a);
    NodePtr tanh(NodePtr a);
    NodePtr sigmoid(NodePtr a);
    NodePtr gelu(NodePtr a);
    NodePtr unary(OpEnum op, NodePtr a);
    NodePtr binary(OpEnum op, NodePtr a, NodePtr b);

    NodePtr matmul(NodePtr A, NodePtr B);

    NodePtr sum(NodePtr x, const std::vector<int>& axes, bool keepdims);
    NodePtr max(NodePtr x, const std::vector<int>& axes, bool keepdims);
    // Index of the first maximum along one axis (or over the flattened tensor
    // when axes is empty), as int64.
    NodePtr argmax(NodePtr x, const std::vector<int>& axes, bool keepdims);

    NodePtr transpose(NodePtr x, const std::vector<int>& axes);
    NodePtr reshape(NodePtr x, const std::vector<int>& shape);
    NodePtr expand(NodePtr x, const std::vector<int>& shape);
    NodePtr cast(NodePtr x, DType dtype);
}
