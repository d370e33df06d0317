// TEST INFRASTRUCTURE — a driver for the reference's own core.
//
// oracle/Makefile.ref compiles this file into two libraries, from the sources
// where they lie under /root/reference:
//   oracle/_ref/libormi_ref.so      l-h-ha/Ormi's core and CPU backend
//                                   (ormi-core/csrc/core/**, backend/cpu/**
//                                   without the OpenBLAS sgemm,
//                                   backend/runtime.cpp, backend/graph_breakers.cpp)
//                                   exactly as they are; the two functions its
//                                   CUDA device would provide (cuda::execute_jit,
//                                   get_cuda_allocator) stay unresolved and are
//                                   never reached on the CPU device.
//   oracle/_ref/libormi_ref_hip.so  the same sources with the HIP device added as
//                                   a maintainer would add it (the enum value, the
//                                   get_allocator case, the execute_graph case),
//                                   plus the HIP glue of ormi_amd/csrc/ormi_core_hip,
//                                   linked against libormi_hip.so.
// Tests run the same program through the reference's execute_graph /
// compute_gradients on the CPU device (the reference's own result), on the HIP
// device (libormi_hip behind the reference's plugin points) and through the
// restated oracle, and compare.
//
// A program: values 0..num_leaves-1 are leaves (host float32, contiguous, with
// a requires_grad flag, uploaded to the device); each op appends one value,
// built with the reference's own op constructors (csrc/core/ops/**). If
// grad_root >= 0, compute_gradients(value grad_root) runs
// (csrc/core/autograd.cpp:24-47). Outputs name values (>= 0) or leaf gradients
// (-1 - leaf); each is realized with execute_graph (csrc/backend/runtime.cpp:
// 13-39), its buffer copied to the host through the device's allocator, and
// written out in the row-major order of its view (ndim -1: the leaf received
// no gradient). device is a DeviceEnum value: 0 CPU, 2 HIP.
#include <algorithm>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <vector>

#include "backend/runtime.h"
#include "core/allocator.h"
#include "core/autograd.h"
#include "core/memory.h"
#include "core/node.h"
#include "core/shape.h"
#include "core/ops/pointwise/add.h"
#include "core/ops/pointwise/cos.h"
#include "core/ops/pointwise/div.h"
#include "core/ops/pointwise/exp.h"
#include "core/ops/pointwise/log.h"
#include "core/ops/pointwise/mul.h"
#include "core/ops/pointwise/neg.h"
#include "core/ops/pointwise/pow.h"
#include "core/ops/pointwise/sin.h"
#include "core/ops/pointwise/sub.h"
#include "core/ops/reduce/sum.h"
#include "core/ops/view/expand.h"
#include "core/ops/view/reshape.h"
#include "core/ops/view/transpose.h"
#include "core/ops/blas/matmul.h"

extern "C" {
// A leaf's buffer holds numel floats (0: the product of its shape). With
// has_strides its view gets the given strides over that buffer, as the
// reference's own tests set a leaf's view (csrc/tests/backend/cpu/kernels/
// blas/test_matmul.cpp:58-62); otherwise it is contiguous.
typedef struct ref_leaf {
    const float* data;
    int ndim;
    int shape[8];
    int requires_grad;
    long long numel;
    int has_strides;
    int strides[8];
} ref_leaf;

// op: 0 NEG 1 EXP 2 LOG 3 SIN 4 COS 5 ADD 6 SUB 7 MUL 8 DIV 9 POW
//     10 SUM(attr = axes, keepdims) 11 TRANSPOSE(attr = axes)
//     12 RESHAPE(attr = shape) 13 EXPAND(attr = shape) 14 MATMUL
typedef struct ref_op {
    int op, a, b;
    int nattr;
    int attr[8];
    int keepdims;
} ref_op;
}

namespace {
    using ormi::Node;
    using NodePtr = std::shared_ptr<Node>;

    NodePtr build_op(const ref_op& o, const std::vector<NodePtr>& v) {
        const NodePtr& a = v.at(o.a);
        const std::vector<int> attr(o.attr, o.attr + std::max(0, std::min(o.nattr, 8)));
        switch (o.op) {
            case 0: return ormi::ops::neg(a);
            case 1: return ormi::ops::exp(a);
            case 2: return ormi::ops::log(a);
            case 3: return ormi::ops::sin(a);
            case 4: return ormi::ops::cos(a);
            case 5: return ormi::ops::add(a, v.at(o.b));
            case 6: return ormi::ops::sub(a, v.at(o.b));
            case 7: return ormi::ops::mul(a, v.at(o.b));
            case 8: return ormi::ops::div(a, v.at(o.b));
            case 9: return ormi::ops::pow(a, v.at(o.b));
            case 10: return ormi::ops::sum(a, attr, o.keepdims != 0);
            case 11: return ormi::ops::transpose(a, attr);
            case 12: return ormi::ops::reshape(a, attr);
            case 13: return ormi::ops::expand(a, attr);
            case 14: return ormi::ops::matmul(a, v.at(o.b));
        }
        throw std::runtime_error("ref_run: unknown op code");
    }

    // Row-major copy of a realized node's view (views alias their parent's
    // buffer with their own strides), read from a host copy of the buffer.
    long long copy_out(const NodePtr& n, float* out, long long cap) {
        const auto& shape = n->view.shape;
        const auto& st = n->view.strides;
        long long count = 1;
        for (int e : shape) count *= e;
        if (count > cap) throw std::runtime_error("ref_run: output buffer too small");
        if (count == 0) return 0;
        std::vector<float> host(n->data->bytes / sizeof(float));
        ormi::get_allocator(n->data->device.type)->copy_device_to_host(host.data(), n->data->ptr, n->data->bytes);
        std::vector<int> idx(shape.size(), 0);
        for (long long i = 0; i < count; ++i) {
            long long off = 0;
            for (size_t d = 0; d < shape.size(); ++d) off += (long long)idx[d] * st[d];
            if (off < 0 || off >= (long long)host.size()) throw std::runtime_error("ref_run: view reads past its buffer");
            out[i] = host[off];
            for (int d = (int)shape.size() - 1; d >= 0; --d) {
                if (++idx[d] < shape[d]) break;
                idx[d] = 0;
            }
        }
        return count;
    }
}

// 1 when the device's allocator can be made, as the reference's test fixture
// probes a device (csrc/tests/test_utils.h:17-21); else 0 and the message the
// allocator threw.
extern "C" __attribute__((visibility("default"))) int ref_device_available(int device, char* err, int err_len) {
    try {
        return ormi::get_allocator(static_cast<ormi::DeviceEnum>(device)) != nullptr ? 1 : 0;
    } catch (const std::exception& e) {
        if (err && err_len > 0) {
            std::strncpy(err, e.what(), (size_t)err_len - 1);
            err[err_len - 1] = '\0';
        }
        return 0;
    }
}

extern "C" __attribute__((visibility("default"))) int ref_run(int device, int num_leaves, const ref_leaf* leaves, int num_ops, const ref_op* ops, int grad_root,
                       int num_outputs, const int* output_ids, float* const* outputs, const long long* capacities,
                       int* out_ndim, int* out_shapes, char* err, int err_len) {
    try {
        const auto dev_type = static_cast<ormi::DeviceEnum>(device);
        const ormi::Device dev(dev_type, 0);
        std::vector<NodePtr> v;
        std::vector<NodePtr> leaf_nodes;
        for (int i = 0; i < num_leaves; ++i) {
            const ref_leaf& L = leaves[i];
            std::vector<int> shape(L.shape, L.shape + L.ndim);
            std::vector<int> buf_shape = shape;
            if (L.numel > 0) buf_shape = {(int)L.numel};
            auto buf = ormi::empty(buf_shape, dev_type);
            if (buf->bytes) ormi::get_allocator(dev_type)->copy_host_to_device(buf->ptr, L.data, buf->bytes);
            auto n = std::make_shared<Node>(buf, L.requires_grad != 0, dev);
            n->view.shape = shape;
            n->view.strides = L.has_strides ? std::vector<int>(L.strides, L.strides + L.ndim)
                                            : ormi::calc_contiguous_strides(shape);
            v.push_back(n);
            leaf_nodes.push_back(n);
        }
        for (int k = 0; k < num_ops; ++k) v.push_back(build_op(ops[k], v));
        if (grad_root >= 0) ormi::compute_gradients(v.at(grad_root));
        for (int o = 0; o < num_outputs; ++o) {
            const int id = output_ids[o];
            NodePtr n = id >= 0 ? v.at(id) : leaf_nodes.at(-1 - id)->grad;
            if (!n) {  // a leaf the gradient does not reach
                out_ndim[o] = -1;
                continue;
            }
            ormi::execute_graph(n);
            out_ndim[o] = (int)n->view.shape.size();
            for (size_t d = 0; d < n->view.shape.size() && d < 8; ++d) out_shapes[8 * o + d] = n->view.shape[d];
            copy_out(n, outputs[o], capacities[o]);
        }
        return 0;
    } catch (const std::exception& e) {
        if (err && err_len > 0) {
            std::strncpy(err, e.what(), (size_t)err_len - 1);
            err[err_len - 1] = '\0';
        }
        return 1;
    }
}
