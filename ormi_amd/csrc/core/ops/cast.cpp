// CAST (additive): element type conversion, materialized contiguously.
// Float -> bf16/fp16 rounds to nearest even. Integer targets (int64, int32,
// bool) convert the float32 value on store: truncation toward zero with NaN
// giving 0 and saturation at the type's range, or x != 0 for bool.
#include <stdexcept>
#include "core/ops/api.h"
#include "core/shape.h"
#include "core/adjoint.h"
#include "core/registry.h"

namespace ormi {
    using ops::OpEnum;
    using NodeVec = std::vector<std::shared_ptr<Node>>;

    namespace ops {
        NodePtr cast(NodePtr x, DType dtype) {
            // A cast to the operand's own type is the operand: nodes are never
            // written after they are realized, so aliasing is invisible, and an
            // int64 value above 2^24 must not round through the fp32 registers
            // the element-wise kernels compute in.
            if (x->dtype == dtype) return x;
            return std::make_shared<Node>(OpEnum::CAST, NodeVec{x}, x->device, CastAttrs{dtype});
        }
    }

    static void adjoint_cast(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (!x->requires_grad) return;
        std::shared_ptr<Node> g = n->grad;
        if (x->dtype != g->dtype) g = std::make_shared<Node>(OpEnum::CAST, NodeVec{g}, n->device, CastAttrs{x->dtype});
        accumulate_grad(x, g, n->device);
    }

    static RegisterShape rs_cast(OpEnum::CAST, infer_unary_shape);
    static RegisterAdjoint ra_cast(OpEnum::CAST, adjoint_cast);
}
