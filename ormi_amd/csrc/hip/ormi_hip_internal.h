// Helpers shared by the translation units of libormi_hip.so (not exported).
#pragma once
#include <string>

namespace ormi_hip {
    // Record msg as the thread's last error and return code.
    int fail(int code, const std::string& msg);
    // Bind device 0 on first use (ormi_hip_init was not called explicitly).
    int ensure_init();
    // Compute units of the bound device (256 on MI355X).
    int compute_units();
}
