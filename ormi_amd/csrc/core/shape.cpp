#include <stdexcept>
#include <algorithm>
#include <climits>
#include <string>
#include "core/shape.h"
#include "core/node.h"

namespace ormi {
    bool TensorView::is_contiguous() const {
        long long expected = 1;
        for (int i = (int)shape.size() - 1; i >= 0; --i) {
            if (strides[i] != expected) return false;
            expected *= shape[i];
        }
        return true;
    }

    int checked_extent(long long v, const char* what) {
        if (v > INT_MAX || v < INT_MIN)
            throw std::runtime_error(std::string(what) + " " + std::to_string(v) +
                                     " exceeds the 32-bit range of TensorView (shapes and strides are int).");
        return (int)v;
    }

    // Strides are computed in 64 bits: a trailing extent product of 2^31 or more
    // (2 x 32768 x 65536, say) is an error, never a wrapped stride.
    std::vector<int> calc_contiguous_strides(const std::vector<int>& shape) {
        std::vector<int> strides(shape.size(), 1);
        long long s = 1;
        for (int i = (int)shape.size() - 2; i >= 0; --i) {
            s *= shape[i + 1];
            strides[i] = checked_extent(s, "Contiguous stride");
        }
        return strides;
    }

    // Right-aligned numpy broadcasting (reference: csrc/core/shape.cpp:27-44).
    // A size-1 dim takes the other operand's size, so a 0-length dim against
    // 1 stays 0 as in numpy; the reference takes max(da, db) = 1 there, and its
    // kernels then read an element of the empty operand.
    std::vector<int> broadcast_shapes(const std::vector<int>& a, const std::vector<int>& b) {
        const int na = (int)a.size(), nb = (int)b.size();
        const int n = std::max(na, nb);
        std::vector<int> out(n);
        for (int i = 0; i < n; ++i) {
            const int da = i < n - na ? 1 : a[i - (n - na)];
            const int db = i < n - nb ? 1 : b[i - (n - nb)];
            if (da != db && da != 1 && db != 1) throw std::runtime_error("Operands could not be broadcast together.");
            out[i] = da == 1 ? db : da;
        }
        return out;
    }

    std::vector<int> infer_shape(ops::OpEnum op, const std::vector<std::shared_ptr<Node>>& parents, const OpAttributes& attrs) {
        if (op == ops::OpEnum::LEAF || op == ops::OpEnum::CONST || parents.empty()) return {};
        const ShapeInferFunc* func = Registry<ShapeInferFunc>::find(op);
        if (!func) throw std::runtime_error("Shape inference rule not registered for this OpEnum.");
        return (*func)(parents, attrs);
    }

    std::vector<int> infer_unary_shape(const std::vector<std::shared_ptr<Node>>& parents, const OpAttributes&) {
        return parents[0]->view.shape;
    }

    std::vector<int> infer_binary_shape(const std::vector<std::shared_ptr<Node>>& parents, const OpAttributes&) {
        return broadcast_shapes(parents[0]->view.shape, parents[1]->view.shape);
    }

    long long shape_numel(const std::vector<int>& shape) {
        long long n = 1;
        for (int d : shape) n *= d;
        return n;
    }
}
