#pragma once
#include <memory>
#include <vector>
#include "core/node.h"

namespace ormi {
    std::shared_ptr<Node> unbroadcast(std::shared_ptr<Node> grad, const std::vector<int>& target_shape);
    // x->grad = x->grad ? x->grad + g : g  (the accumulation every reference adjoint repeats)
    void accumulate_grad(const std::shared_ptr<Node>& x, const std::shared_ptr<Node>& g, const Device& dev);
}
