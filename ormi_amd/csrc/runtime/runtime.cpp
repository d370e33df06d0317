#include <map>
#include <stdexcept>
#include <unordered_set>
#include <vector>
#include "runtime/runtime.h"
#include "runtime/graph_breakers.h"
#include "core/registry.h"

namespace ormi {
    static std::map<DeviceEnum, JitFunc>& jit_table() { static std::map<DeviceEnum, JitFunc> t; return t; }
    static std::map<DeviceEnum, SchedulerFunc>& sched_table() { static std::map<DeviceEnum, SchedulerFunc> t; return t; }

    static std::map<DeviceEnum, GroupSchedulerFunc>& group_table() { static std::map<DeviceEnum, GroupSchedulerFunc> t; return t; }

    void register_jit(DeviceEnum d, JitFunc f) { jit_table()[d] = std::move(f); }
    void register_group_scheduler(DeviceEnum d, GroupSchedulerFunc f) { group_table()[d] = std::move(f); }
    void register_scheduler(DeviceEnum d, SchedulerFunc f) { sched_table()[d] = std::move(f); }
    bool has_jit(DeviceEnum d) { return jit_table().count(d) > 0; }

    void run_jit(std::shared_ptr<Node> root) {
        auto it = jit_table().find(root->device.type);
        if (it == jit_table().end()) throw std::runtime_error("FATAL: Unsupported device for JIT compiler.");
        it->second(root);
    }

    bool is_view_op(ops::OpEnum op) { return ViewOpRegistry::get().contains(op); }

    static void realize_one(const std::shared_ptr<Node>& node) {
        if (is_view_op(node->op)) {
            node->data = node->parents[0]->data;
            return;
        }
        if (try_execute_graph_break(node)) return;
        auto it = jit_table().find(node->device.type);
        if (it == jit_table().end()) throw std::runtime_error("FATAL: Unsupported device for JIT compiler.");
        it->second(node);
    }

    // Post-order over the unrealized part of the graph: every parent is realized
    // before its child, exactly the order of the reference's recursion, without
    // recursion depth limits.
    void execute_graph_eager(std::shared_ptr<Node> root) {
        if (!root || root->is_realized()) return;
        std::unordered_set<Node*> visited{root.get()};
        std::vector<std::pair<std::shared_ptr<Node>, size_t>> stack{{root, 0}};
        while (!stack.empty()) {
            auto& [node, next] = stack.back();
            if (next < node->parents.size()) {
                auto p = node->parents[next++];
                if (!p->is_realized() && visited.insert(p.get()).second) stack.push_back({p, 0});
            } else {
                auto n = node;
                stack.pop_back();
                realize_one(n);
            }
        }
    }

    void execute_graph(std::shared_ptr<Node> root) {
        if (!root || root->is_realized()) return;
        auto it = sched_table().find(root->device.type);
        if (it != sched_table().end()) it->second(root);
        else execute_graph_eager(root);
    }

    void execute_graph_group(const std::vector<std::shared_ptr<Node>>& roots) {
        std::map<DeviceEnum, std::vector<std::shared_ptr<Node>>> by_device;
        std::vector<DeviceEnum> order;
        for (const auto& r : roots) {
            if (!r || r->is_realized()) continue;
            auto& v = by_device[r->device.type];
            if (v.empty()) order.push_back(r->device.type);
            v.push_back(r);
        }
        for (DeviceEnum d : order) {
            auto it = group_table().find(d);
            if (it != group_table().end()) it->second(by_device[d]);
            else
                for (const auto& r : by_device[d]) execute_graph(r);
        }
    }
}
