#include "core/adjoint.h"
#include "core/shape.h"

namespace ormi {
    // Sum a broadcast gradient back to target_shape (reference: csrc/core/adjoint.cpp:5-34):
    // leading extra axes and axes stretched from 1 are reduced, and the SUM
    // node's view is then set to target_shape (which keeps its 1-sized axes).
    std::shared_ptr<Node> unbroadcast(std::shared_ptr<Node> grad, const std::vector<int>& target_shape) {
        if (grad->view.shape == target_shape) return grad;
        const int ng = (int)grad->view.shape.size(), nt = (int)target_shape.size();
        std::vector<int> axes;
        for (int i = 0; i < ng - nt; ++i) axes.push_back(i);
        for (int i = ng - nt; i < ng; ++i) {
            if (target_shape[i - (ng - nt)] == 1 && grad->view.shape[i] > 1) axes.push_back(i);
        }
        if (axes.empty()) return grad;
        ReduceAttrs attrs;
        attrs.axes = axes;
        attrs.keepdims = false;
        auto s = std::make_shared<Node>(ops::OpEnum::SUM, std::vector<std::shared_ptr<Node>>{grad}, grad->device, attrs);
        s->view.shape = target_shape;
        s->view.strides = calc_contiguous_strides(target_shape);
        return s;
    }

    void accumulate_grad(const std::shared_ptr<Node>& x, const std::shared_ptr<Node>& g, const Device& dev) {
        if (!x->grad) x->grad = g;
        else x->grad = std::make_shared<Node>(ops::OpEnum::ADD, std::vector<std::shared_ptr<Node>>{x->grad, g}, dev);
    }
}
