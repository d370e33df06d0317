#pragma once
#include <unordered_map>
#include <unordered_set>
#include <functional>
#include <vector>
#include <memory>
#include "core/ops.h"
#include "core/attributes.h"

namespace ormi {
    struct Node;

    using ShapeInferFunc  = std::function<std::vector<int>(const std::vector<std::shared_ptr<Node>>&, const OpAttributes&)>;
    using StrideInferFunc = std::function<std::vector<int>(const std::vector<std::shared_ptr<Node>>&, const OpAttributes&, const std::vector<int>& out_shape)>;
    using AdjointFunc     = std::function<void(std::shared_ptr<Node>)>;

    // Per-op rule tables, same shape as the reference's (csrc/core/registry.h:19-37).
    // get_map() is defined once in libormi_core.so (registry.cpp) so that every
    // shared object that registers rules (the core, the test-only CPU oracle)
    // sees the same table.
    template <typename FuncType>
    class Registry {
    public:
        static std::unordered_map<ops::OpEnum, FuncType>& get_map();
        static void add(ops::OpEnum op, FuncType func) { get_map()[op] = std::move(func); }
        static FuncType get(ops::OpEnum op) {
            const FuncType* f = find(op);
            return f ? *f : FuncType(nullptr);
        }
        // The registered rule, or nullptr (no copy of the function object).
        static const FuncType* find(ops::OpEnum op) {
            auto& m = get_map();
            auto it = m.find(op);
            return it == m.end() || !it->second ? nullptr : &it->second;
        }
    };

    class ViewOpRegistry {
    public:
        static ViewOpRegistry& get();
        void add(ops::OpEnum op) { ops_.insert(op); }
        bool contains(ops::OpEnum op) const { return ops_.count(op) > 0; }
    private:
        std::unordered_set<ops::OpEnum> ops_;
    };

    struct RegisterViewOp { explicit RegisterViewOp(ops::OpEnum op) { ViewOpRegistry::get().add(op); } };
    struct RegisterShape  { RegisterShape(ops::OpEnum op, ShapeInferFunc f) { Registry<ShapeInferFunc>::add(op, std::move(f)); } };
    struct RegisterStride { RegisterStride(ops::OpEnum op, StrideInferFunc f) { Registry<StrideInferFunc>::add(op, std::move(f)); } };
    struct RegisterAdjoint{ RegisterAdjoint(ops::OpEnum op, AdjointFunc f) { Registry<AdjointFunc>::add(op, std::move(f)); } };
}
