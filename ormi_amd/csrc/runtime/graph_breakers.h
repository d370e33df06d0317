#pragma once
#include <functional>
#include <memory>
#include "core/node.h"

namespace ormi {
    // (device, op) -> handler that must set root->data to a buffer shaped like
    // root->view.shape (reference: csrc/backend/graph_breakers.h:8-14).
    using GraphBreakHandler = std::function<void(std::shared_ptr<Node>)>;

    bool try_execute_graph_break(std::shared_ptr<Node> root);
    bool has_graph_breaker(DeviceEnum dev, ops::OpEnum op);

    struct RegisterGraphBreaker {
        RegisterGraphBreaker(DeviceEnum dev, ops::OpEnum op, GraphBreakHandler handler);
    };
}
