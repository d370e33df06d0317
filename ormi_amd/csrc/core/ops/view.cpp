// Zero-copy views: TRANSPOSE, RESHAPE, EXPAND (reference: csrc/core/ops/view/
// transpose.cpp:12-73, reshape.cpp:12-97, expand.cpp:13-67). A view node's
// buffer is its parent's buffer; only shape and strides change.
#include <stdexcept>
#include "core/ops/api.h"
#include "core/shape.h"
#include "core/adjoint.h"
#include "core/registry.h"

namespace ormi {
    using ops::OpEnum;
    using NodeVec = std::vector<std::shared_ptr<Node>>;

    namespace ops {
        NodePtr transpose(NodePtr x, const std::vector<int>& axes) {
            return std::make_shared<Node>(OpEnum::TRANSPOSE, NodeVec{x}, x->device, PermuteAttrs{axes});
        }
        NodePtr reshape(NodePtr x, const std::vector<int>& shape) {
            return std::make_shared<Node>(OpEnum::RESHAPE, NodeVec{x}, x->device, ReshapeAttrs{shape});
        }
        NodePtr expand(NodePtr x, const std::vector<int>& shape) {
            return std::make_shared<Node>(OpEnum::EXPAND, NodeVec{x}, x->device, ExpandAttrs{shape});
        }
    }

    // ---- TRANSPOSE: out[i] = in[axes[i]] for shape and strides.
    static std::vector<int> infer_transpose_shape(const NodeVec& parents, const OpAttributes& attrs) {
        if (parents.empty()) throw std::runtime_error("TRANSPOSE requires 1 parent.");
        const auto& in = parents[0]->view.shape;
        const auto& axes = std::get<PermuteAttrs>(attrs).axes;
        if (in.size() != axes.size()) throw std::runtime_error("TRANSPOSE axes count must match tensor dimensions.");
        std::vector<int> seen(in.size(), 0), out(in.size());
        for (size_t i = 0; i < axes.size(); ++i) {
            if (axes[i] < 0 || axes[i] >= (int)in.size() || seen[axes[i]]++) throw std::runtime_error("TRANSPOSE axes must be a permutation.");
            out[i] = in[axes[i]];
        }
        return out;
    }
    static std::vector<int> infer_transpose_strides(const NodeVec& parents, const OpAttributes& attrs, const std::vector<int>&) {
        const auto& axes = std::get<PermuteAttrs>(attrs).axes;
        std::vector<int> out(axes.size());
        for (size_t i = 0; i < axes.size(); ++i) out[i] = parents[0]->view.strides[axes[i]];
        return out;
    }
    static void adjoint_transpose(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (!x->requires_grad) return;
        const auto& axes = std::get<PermuteAttrs>(n->attrs).axes;
        std::vector<int> inv(axes.size());
        for (size_t i = 0; i < axes.size(); ++i) inv[axes[i]] = (int)i;
        accumulate_grad(x, std::make_shared<Node>(OpEnum::TRANSPOSE, NodeVec{n->grad}, n->device, PermuteAttrs{inv}), n->device);
    }

    // ---- RESHAPE: zero-copy only. Old and new dims are matched in blocks of
    // equal element count; each old block must be laid out contiguously (size-1
    // dims exempt), and the new block's strides grow from the old block's
    // innermost stride. Trailing new 1-sized dims get stride 1.
    static std::vector<int> infer_reshape_shape(const NodeVec& parents, const OpAttributes& attrs) {
        if (parents.empty()) throw std::runtime_error("RESHAPE requires 1 parent.");
        return std::get<ReshapeAttrs>(attrs).shape;
    }
    static std::vector<int> infer_reshape_strides(const NodeVec& parents, const OpAttributes&, const std::vector<int>& out) {
        const auto& old_shape = parents[0]->view.shape;
        const auto& old_strides = parents[0]->view.strides;
        if (shape_numel(old_shape) != shape_numel(out)) throw std::runtime_error("RESHAPE size mismatch.");
        if (old_shape.empty()) return calc_contiguous_strides(out);
        std::vector<int> strides(out.size(), 0);
        size_t o = 0, n = 0;
        while (o < old_shape.size() && n < out.size()) {
            size_t o_end = o + 1, n_end = n + 1;
            long long old_prod = old_shape[o], new_prod = out[n];
            while (old_prod != new_prod) {
                if (old_prod < new_prod) {
                    if (o_end >= old_shape.size()) throw std::runtime_error("RESHAPE size mismatch.");
                    old_prod *= old_shape[o_end++];
                } else {
                    if (n_end >= out.size()) throw std::runtime_error("RESHAPE size mismatch.");
                    new_prod *= out[n_end++];
                }
            }
            for (size_t i = o; i + 1 < o_end; ++i) {
                if (old_shape[i] != 1 && old_shape[i + 1] != 1 &&
                    (long long)old_strides[i] != (long long)old_shape[i + 1] * old_strides[i + 1])
                    throw std::runtime_error("RESHAPE cannot be performed as a zero-copy view because the tensor is not contiguous across merged dimensions.");
            }
            long long s = old_strides[o_end - 1];
            for (size_t i = n_end; i-- > n;) {
                strides[i] = checked_extent(s, "RESHAPE stride");
                s *= out[i];
            }
            o = o_end;
            n = n_end;
        }
        for (; o < old_shape.size(); ++o)
            if (old_shape[o] != 1) throw std::runtime_error("RESHAPE size mismatch trailing dims.");
        for (; n < out.size(); ++n) {
            if (out[n] != 1) throw std::runtime_error("RESHAPE size mismatch trailing dims.");
            strides[n] = 1;
        }
        return strides;
    }
    static void adjoint_reshape(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (!x->requires_grad) return;
        accumulate_grad(x, std::make_shared<Node>(OpEnum::RESHAPE, NodeVec{n->grad}, n->device, ReshapeAttrs{x->view.shape}), n->device);
    }

    // ---- EXPAND: right-aligned; new leading dims and stretched 1-dims get stride 0.
    static std::vector<int> infer_expand_shape(const NodeVec& parents, const OpAttributes& attrs) {
        if (parents.empty()) throw std::runtime_error("EXPAND requires 1 parent.");
        const auto& in = parents[0]->view.shape;
        const auto& out = std::get<ExpandAttrs>(attrs).shape;
        if (out.size() < in.size()) throw std::runtime_error("EXPAND cannot drop dimensions.");
        const size_t off = out.size() - in.size();
        for (size_t i = 0; i < in.size(); ++i)
            if (in[i] != 1 && in[i] != out[off + i]) throw std::runtime_error("EXPAND target shape is incompatible.");
        return out;
    }
    static std::vector<int> infer_expand_strides(const NodeVec& parents, const OpAttributes&, const std::vector<int>& out) {
        const auto& ps = parents[0]->view.shape;
        const auto& pst = parents[0]->view.strides;
        const int off = (int)out.size() - (int)ps.size();
        std::vector<int> strides(out.size(), 0);
        for (int i = off; i < (int)out.size(); ++i) {
            const int d = i - off;
            strides[i] = (ps[d] == 1 && out[i] > 1) ? 0 : pst[d];
        }
        return strides;
    }
    static void adjoint_expand(std::shared_ptr<Node> n) {
        auto x = n->parents[0];
        if (!x->requires_grad) return;
        accumulate_grad(x, unbroadcast(n->grad, x->view.shape), n->device);
    }

    static RegisterShape rs_t(OpEnum::TRANSPOSE, infer_transpose_shape);
    static RegisterStride rst_t(OpEnum::TRANSPOSE, infer_transpose_strides);
    static RegisterAdjoint ra_t(OpEnum::TRANSPOSE, adjoint_transpose);
    static RegisterViewOp rv_t(OpEnum::TRANSPOSE);
    static RegisterShape rs_r(OpEnum::RESHAPE, infer_reshape_shape);
    static RegisterStride rst_r(OpEnum::RESHAPE, infer_reshape_strides);
    static RegisterAdjoint ra_r(OpEnum::RESHAPE, adjoint_reshape);
    static RegisterViewOp rv_r(OpEnum::RESHAPE);
    static RegisterShape rs_e(OpEnum::EXPAND, infer_expand_shape);
    static RegisterStride rst_e(OpEnum::EXPAND, infer_expand_strides);
    static RegisterAdjoint ra_e(OpEnum::EXPAND, adjoint_expand);
    static RegisterViewOp rv_e(OpEnum::EXPAND);
}
