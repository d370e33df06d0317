#pragma once
#include <memory>
#include <vector>
#include "core/node.h"

namespace ormi {
    void compute_gradients(std::shared_ptr<Node> root);
    void zero_grad_graph(std::shared_ptr<Node> root);
    // Post-order (parents before children) list of every node reachable from root.
    std::vector<std::shared_ptr<Node>> topo_order(const std::shared_ptr<Node>& root);
}
