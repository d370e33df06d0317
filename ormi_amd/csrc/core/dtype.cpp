#include <stdexcept>
#include "core/dtype.h"

namespace ormi {
    size_t dtype_size(DType dtype) {
        switch (dtype) {
            case DType::Float32: return 4;
            case DType::Int32:   return 4;
            case DType::Bool:    return 1;
            case DType::BFloat16:return 2;
            case DType::Float16: return 2;
            case DType::Int64:   return 8;
        }
        throw std::runtime_error("Unsupported DType.");
    }

    const char* dtype_name(DType dtype) {
        switch (dtype) {
            case DType::Float32: return "float32";
            case DType::Int32:   return "int32";
            case DType::Bool:    return "bool";
            case DType::BFloat16:return "bfloat16";
            case DType::Float16: return "float16";
            case DType::Int64:   return "int64";
        }
        throw std::runtime_error("Unsupported DType.");
    }

    DType dtype_from_name(const std::string& n) {
        if (n == "float32" || n == "f32") return DType::Float32;
        if (n == "int32" || n == "i32") return DType::Int32;
        if (n == "bool") return DType::Bool;
        if (n == "bfloat16" || n == "bf16") return DType::BFloat16;
        if (n == "float16" || n == "f16" || n == "half") return DType::Float16;
        if (n == "int64" || n == "i64") return DType::Int64;
        throw std::runtime_error("Unknown dtype name: " + n);
    }
}
