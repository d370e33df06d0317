// The element-wise tape of an ormi_map_desc as the code generator's Expr:
// shared by ormi_hip_map (map_entry.cpp) and ormi_hip_reduce_map, whose
// reduction evaluates the tape as its prologue (reduce_entry.cpp). Not
// exported.
#pragma once
#include <vector>

#include "backend/hip/kernel_gen.h"
#include "ormi_hip.h"

namespace ormi_hip {
    struct MapTape {
        ormi::hip::Expr expr;  // roots: the output values, in output order
        std::vector<int> shape;
        std::vector<void*> outs;               // with_buffers only
        std::vector<ormi::DType> out_dtypes;   // with_buffers only
        long long numel = 1;
    };

    // Checks d and builds the tape; on a bad descriptor records "<who>: <why>"
    // as the last error and returns ORMI_HIP_ERR_INVALID. with_buffers: every
    // output names a buffer and a dtype (ormi_hip_map); otherwise only the
    // output values are read.
    int parse_map_tape(const ormi_map_desc* d, const char* who, bool with_buffers, MapTape* t);
}
