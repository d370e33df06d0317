#pragma once
#include <cstddef>
#include <cstdint>
#include <string>

namespace ormi {
    // Element types a Buffer can hold. The first three keep the numbering of the
    // reference enum (csrc/core/dtype.h:4-8); the rest are additive for the
    // bf16 GEMM inputs and the int64 argmax output.
    enum class DType { Float32, Int32, Bool, BFloat16, Float16, Int64 };

    size_t dtype_size(DType dtype);
    const char* dtype_name(DType dtype);
    DType dtype_from_name(const std::string& name);
}
