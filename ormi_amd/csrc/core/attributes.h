#pragma once
#include <vector>
#include <variant>
#include "core/dtype.h"

namespace ormi {
    struct NoAttrs {};

    struct ReduceAttrs {
        std::vector<int> axes;     // empty = reduce every axis
        bool keepdims = false;
    };

    struct PermuteAttrs { std::vector<int> axes; };
    struct ReshapeAttrs { std::vector<int> shape; };
    struct ExpandAttrs  { std::vector<int> shape; };
    struct CastAttrs    { DType dtype = DType::Float32; };

    using OpAttributes = std::variant<NoAttrs, ReduceAttrs, PermuteAttrs, ReshapeAttrs, ExpandAttrs, CastAttrs>;
}
