#pragma once
#include <vector>
#include <memory>
#include "core/shape.h"
#include "core/ops.h"
#include "core/device.h"
#include "core/memory.h"
#include "core/attributes.h"

namespace ormi {
    // One vertex of the lazy graph (reference: csrc/core/node.h:12-37).
    // dtype (additive) is the element type the node's buffer holds once realized.
    struct Node : public std::enable_shared_from_this<Node> {
        ops::OpEnum op;
        std::vector<std::shared_ptr<Node>> parents;
        std::shared_ptr<Buffer> data;
        std::shared_ptr<Node> grad;
        bool requires_grad = false;
        Device device;
        TensorView view;
        OpAttributes attrs;
        DType dtype = DType::Float32;

        Node(std::shared_ptr<Buffer> mem, bool req_grad, Device dev);
        Node(ops::OpEnum operation, std::vector<std::shared_ptr<Node>> parent_nodes, Device dev,
             OpAttributes attributes = NoAttrs{});

        bool is_realized() const;
        void realize();
    };
}
