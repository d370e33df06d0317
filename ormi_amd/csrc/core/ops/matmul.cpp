// MATMUL (reference: csrc/core/ops/blas/matmul.cpp:14-138): batch dims broadcast,
// the last two dims multiply; the adjoint issues dX = dZ.Y^T and dY = X^T.dZ
// through zero-copy TRANSPOSE views.
#include <stdexcept>
#include <algorithm>
#include "core/ops/api.h"
#include "core/shape.h"
#include "core/adjoint.h"
#include "core/registry.h"

namespace ormi {
    using ops::OpEnum;
    using NodeVec = std::vector<std::shared_ptr<Node>>;

    namespace ops {
        NodePtr matmul(NodePtr A, NodePtr B) {
            if (!A || !B) throw std::runtime_error("MATMUL got a null operand.");
            if (A->device.type != B->device.type) throw std::runtime_error("Device mismatch in MatMul.");
            return std::make_shared<Node>(OpEnum::MATMUL, NodeVec{A, B}, A->device);
        }
    }

    static std::vector<int> infer_matmul_shape(const NodeVec& parents, const OpAttributes&) {
        if (parents.size() < 2) throw std::runtime_error("MATMUL requires 2 parents.");
        const auto& a = parents[0]->view.shape;
        const auto& b = parents[1]->view.shape;
        const int na = (int)a.size(), nb = (int)b.size();
        if (na < 2 || nb < 2) throw std::runtime_error("MATMUL requires operands to have at least 2 dimensions.");
        if (a[na - 1] != b[nb - 2]) throw std::runtime_error("MATMUL inner dimensions must match (K_a != K_b).");
        std::vector<int> out;
        if (na > 2 || nb > 2) {
            try {
                out = broadcast_shapes(std::vector<int>(a.begin(), a.end() - 2), std::vector<int>(b.begin(), b.end() - 2));
            } catch (const std::runtime_error&) {
                throw std::runtime_error("MATMUL batch dimensions could not be broadcast together.");
            }
        }
        out.push_back(a[na - 2]);
        out.push_back(b[nb - 1]);
        return out;
    }

    static std::vector<int> swap_last_two(int ndim) {
        std::vector<int> axes(ndim);
        for (int i = 0; i < ndim; ++i) axes[i] = i;
        if (ndim >= 2) std::swap(axes[ndim - 2], axes[ndim - 1]);
        return axes;
    }

    static void adjoint_matmul(std::shared_ptr<Node> n) {
        auto dz = n->grad;
        auto x = n->parents[0], y = n->parents[1];
        if (x->requires_grad) {
            auto yt = std::make_shared<Node>(OpEnum::TRANSPOSE, NodeVec{y}, n->device, PermuteAttrs{swap_last_two((int)y->view.shape.size())});
            auto g = std::make_shared<Node>(OpEnum::MATMUL, NodeVec{dz, yt}, n->device);
            accumulate_grad(x, unbroadcast(g, x->view.shape), n->device);
        }
        if (y->requires_grad) {
            auto xt = std::make_shared<Node>(OpEnum::TRANSPOSE, NodeVec{x}, n->device, PermuteAttrs{swap_last_two((int)x->view.shape.size())});
            auto g = std::make_shared<Node>(OpEnum::MATMUL, NodeVec{xt, dz}, n->device);
            accumulate_grad(y, unbroadcast(g, y->view.shape), n->device);
        }
    }

    static RegisterShape rs_matmul(OpEnum::MATMUL, infer_matmul_shape);
    static RegisterAdjoint ra_matmul(OpEnum::MATMUL, adjoint_matmul);
}
