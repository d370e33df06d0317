#pragma once
#include <functional>
#include <memory>
#include <vector>
#include "core/node.h"

namespace ormi {
    // Realize root (reference: csrc/backend/runtime.cpp:13-39). A device that
    // registered a scheduler decides itself which nodes get buffers (the HIP
    // device fuses pointwise regions); every other device gets the reference
    // order: all parents first, views alias, graph breakers, else the device JIT.
    void execute_graph(std::shared_ptr<Node> root);

    // The reference order, for any device (the HIP scheduler never calls it).
    void execute_graph_eager(std::shared_ptr<Node> root);

    bool is_view_op(ops::OpEnum op);

    using JitFunc = std::function<void(std::shared_ptr<Node>)>;
    using SchedulerFunc = std::function<void(std::shared_ptr<Node>)>;

    // Per-device element-wise JIT, the reference's switch (runtime.cpp:29-38) as a table.
    using GroupSchedulerFunc = std::function<void(const std::vector<std::shared_ptr<Node>>&)>;

    void register_jit(DeviceEnum dev, JitFunc fn);
    void register_scheduler(DeviceEnum dev, SchedulerFunc fn);
    // A device may realize several requested nodes together (the HIP device
    // fuses same-shape element-wise roots into one multi-output kernel).
    void register_group_scheduler(DeviceEnum dev, GroupSchedulerFunc fn);

    // Realize every node of roots. Nodes of a device with a group scheduler go
    // to it together (in order); the others are realized one by one.
    void execute_graph_group(const std::vector<std::shared_ptr<Node>>& roots);
    bool has_jit(DeviceEnum dev);
    // Call the registered element-wise JIT of root's device directly.
    void run_jit(std::shared_ptr<Node> root);

    struct RegisterJit { RegisterJit(DeviceEnum d, JitFunc f) { register_jit(d, std::move(f)); } };
    struct RegisterScheduler { RegisterScheduler(DeviceEnum d, SchedulerFunc f) { register_scheduler(d, std::move(f)); } };
    struct RegisterGroupScheduler {
        RegisterGroupScheduler(DeviceEnum d, GroupSchedulerFunc f) { register_group_scheduler(d, std::move(f)); }
    };
}
