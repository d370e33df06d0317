// The HIP device of Ormi's own C++ core (ormi-core/csrc), as a maintainer adds
// it under csrc/backend/hip/: the glue between the reference's plugin points
// and libormi_hip.so's C ABI (include/ormi_hip.h). Nothing here includes a
// HIP header; every device call goes through the C ABI.
//
// HIP_SAFE_CALL plays the part of CUDA_SAFE_CALL (csrc/utils/macros.h:12-18):
// a failing call throws std::runtime_error with the library's message.
#pragma once
#include <stdexcept>
#include <string>

#include "ormi_hip.h"

#define HIP_SAFE_CALL(x)                                                                       \
    do {                                                                                       \
        if ((x) != ORMI_HIP_OK) throw std::runtime_error(std::string("HIP Error: ") + ormi_hip_last_error()); \
    } while (0)
