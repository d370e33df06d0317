#include <map>
#include <mutex>
#include <stdexcept>
#include <unordered_set>
#include <vector>
#include "core/autograd.h"
#include "core/registry.h"
#include "core/memory.h"

namespace ormi {
    // Post-order DFS with an explicit stack; the visiting order matches the
    // reference's recursive build_topo (csrc/core/autograd.cpp:12-22) without
    // its recursion-depth limit.
    std::vector<std::shared_ptr<Node>> topo_order(const std::shared_ptr<Node>& root) {
        std::vector<std::shared_ptr<Node>> topo;
        if (!root) return topo;
        std::unordered_set<Node*> visited;
        std::vector<std::pair<std::shared_ptr<Node>, size_t>> stack;
        visited.insert(root.get());
        stack.push_back({root, 0});
        while (!stack.empty()) {
            auto& [node, next] = stack.back();
            if (next < node->parents.size()) {
                auto p = node->parents[next++];
                if (p && !visited.count(p.get())) {
                    visited.insert(p.get());
                    stack.push_back({p, 0});
                }
            } else {
                topo.push_back(node);
                stack.pop_back();
            }
        }
        return topo;
    }

    // The seed of a one-element root (a loss): one read-only buffer of 1.0 per
    // (device, shape), shared by every backward instead of a fresh allocation
    // and fill launch each time, as Python-scalar leaves are shared. Never
    // freed (device memory outlives static destructors otherwise).
    static std::shared_ptr<Buffer> scalar_seed(const std::vector<int>& shape, DeviceEnum dev) {
        static std::mutex mu;
        static auto* cache = new std::map<std::pair<int, std::vector<int>>, std::shared_ptr<Buffer>>();
        std::lock_guard<std::mutex> lock(mu);
        auto& b = (*cache)[{(int)dev, shape}];
        if (!b) b = ones(shape, dev);
        return b;
    }

    // Reverse-mode pass that only builds lazy gradient nodes
    // (reference: csrc/core/autograd.cpp:24-47).
    void compute_gradients(std::shared_ptr<Node> root) {
        auto topo = topo_order(root);
        if (!root->grad) {
            long long n = 1;
            for (int d : root->view.shape) n *= d;
            auto seed = n == 1 ? scalar_seed(root->view.shape, root->device.type) : ones(root->view.shape, root->device.type);
            root->grad = std::make_shared<Node>(seed, false, root->device);
        }
        for (auto it = topo.rbegin(); it != topo.rend(); ++it) {
            auto node = *it;
            if (!node->grad || node->op == ops::OpEnum::LEAF) continue;
            auto adjoint = Registry<AdjointFunc>::get(node->op);
            if (!adjoint) throw std::runtime_error("No Adjoint rule registered for operation.");
            adjoint(node);
        }
    }

    void zero_grad_graph(std::shared_ptr<Node> root) {
        for (auto& node : topo_order(root)) node->grad = nullptr;
    }
}
