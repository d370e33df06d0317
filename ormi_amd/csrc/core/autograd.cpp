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
    // its recursion-depth limit. Raw pointers: root keeps every node it reaches
    // alive for the walk (no reference-count traffic per step).
    // The visited set is a plain array while the graph is small (a training
    // step's graph is tens of nodes: a linear scan beats hashing and its
    // per-insert allocations) and a hash set past kLinear nodes.
    namespace {
        struct VisitedSet {
            static constexpr size_t kLinear = 48;
            std::vector<Node*> small;
            std::unordered_set<Node*> big;
            VisitedSet() { small.reserve(kLinear); }
            bool insert(Node* n) {  // true when n was not in the set
                if (big.empty()) {
                    for (Node* m : small)
                        if (m == n) return false;
                    if (small.size() < kLinear) {
                        small.push_back(n);
                        return true;
                    }
                    big.reserve(4 * kLinear);
                    big.insert(small.begin(), small.end());
                }
                return big.insert(n).second;
            }
        };
    }

    static std::vector<Node*> topo_nodes(Node* root) {
        std::vector<Node*> topo;
        if (!root) return topo;
        topo.reserve(32);
        VisitedSet visited;
        std::vector<std::pair<Node*, size_t>> stack;
        stack.reserve(32);
        visited.insert(root);
        stack.push_back({root, 0});
        while (!stack.empty()) {
            auto& [node, next] = stack.back();
            if (next < node->parents.size()) {
                Node* p = node->parents[next++].get();
                if (p && visited.insert(p)) stack.push_back({p, 0});
            } else {
                topo.push_back(node);
                stack.pop_back();
            }
        }
        return topo;
    }

    std::vector<std::shared_ptr<Node>> topo_order(const std::shared_ptr<Node>& root) {
        std::vector<std::shared_ptr<Node>> topo;
        for (Node* n : topo_nodes(root.get())) topo.push_back(n->shared_from_this());
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
        const auto topo = topo_nodes(root.get());
        if (!root->grad) {
            long long n = 1;
            for (int d : root->view.shape) n *= d;
            auto seed = n == 1 ? scalar_seed(root->view.shape, root->device.type) : ones(root->view.shape, root->device.type);
            root->grad = std::make_shared<Node>(seed, false, root->device);
        }
        const auto& rules = Registry<AdjointFunc>::get_map();
        for (auto it = topo.rbegin(); it != topo.rend(); ++it) {
            Node* node = *it;
            if (!node->grad || node->op == ops::OpEnum::LEAF) continue;
            auto rule = rules.find(node->op);
            if (rule == rules.end() || !rule->second) throw std::runtime_error("No Adjoint rule registered for operation.");
            rule->second(node->shared_from_this());
        }
    }

    void zero_grad_graph(std::shared_ptr<Node> root) {
        for (Node* node : topo_nodes(root.get())) node->grad = nullptr;
    }
}
