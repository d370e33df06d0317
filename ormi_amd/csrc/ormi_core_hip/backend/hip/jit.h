// hip::execute_jit, the HIP case of execute_graph's device switch
// (csrc/backend/runtime.cpp:29-38), declared as cuda::execute_jit is
// (csrc/backend/cuda/jit.cuh:5-7).
#pragma once
#include <memory>

#include "core/node.h"

namespace ormi::hip {
    void execute_jit(std::shared_ptr<Node> root);
}
