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
    // Resolve the device address of the allocation-free GEMM's scratch array on
    // the current device (called once, by ormi_hip_init).
    int gemm_scratch_setup();
    // Wait until the launch queue has issued every launch submitted so far;
    // returns the error of a queued launch that failed (once).
    int drain_queue();
}
