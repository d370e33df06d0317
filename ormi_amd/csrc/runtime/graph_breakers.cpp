#include <map>
#include "runtime/graph_breakers.h"

namespace ormi {
    static std::map<std::pair<DeviceEnum, ops::OpEnum>, GraphBreakHandler>& breaker_table() {
        static std::map<std::pair<DeviceEnum, ops::OpEnum>, GraphBreakHandler> table;
        return table;
    }

    RegisterGraphBreaker::RegisterGraphBreaker(DeviceEnum dev, ops::OpEnum op, GraphBreakHandler handler) {
        breaker_table()[{dev, op}] = std::move(handler);
    }

    bool has_graph_breaker(DeviceEnum dev, ops::OpEnum op) {
        return breaker_table().count({dev, op}) > 0;
    }

    bool try_execute_graph_break(std::shared_ptr<Node> root) {
        auto& t = breaker_table();
        auto it = t.find({root->device.type, root->op});
        if (it == t.end()) return false;
        it->second(root);
        return true;
    }
}
