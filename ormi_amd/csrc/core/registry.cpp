#include "core/registry.h"

namespace ormi {
    template <typename FuncType>
    std::unordered_map<ops::OpEnum, FuncType>& Registry<FuncType>::get_map() {
        static std::unordered_map<ops::OpEnum, FuncType> map;
        return map;
    }

    template class Registry<ShapeInferFunc>;
    template class Registry<StrideInferFunc>;
    template class Registry<AdjointFunc>;

    ViewOpRegistry& ViewOpRegistry::get() {
        static ViewOpRegistry instance;
        return instance;
    }
}
