// pybind11 module `ormi_backend`: the reference's Python surface
// (csrc/bindings/main.cpp:19-36 and bind_*.cpp) plus the HIP device, dtypes
// and the additive ops.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cmath>
#include <cstring>
#include <optional>

#include "backend/hip/hip_backend.h"
#include "core/allocator.h"
#include "core/autograd.h"
#include "core/memory.h"
#include "core/node.h"
#include "core/ops/api.h"
#include "runtime/graph_breakers.h"
#include "runtime/runtime.h"

namespace py = pybind11;
using namespace ormi;

namespace {
    uint16_t f32_to_bf16_rne(float f) {
        uint32_t u;
        std::memcpy(&u, &f, 4);
        if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
        u += 0x7fffu + ((u >> 16) & 1u);
        return (uint16_t)(u >> 16);
    }

    float bf16_to_f32(uint16_t h) {
        uint32_t u = (uint32_t)h << 16;
        float f;
        std::memcpy(&f, &u, 4);
        return f;
    }

    // IEEE binary16 from binary32, round to nearest even.
    uint16_t f32_to_f16_rne(float f) {
        uint32_t x;
        std::memcpy(&x, &f, 4);
        const uint32_t sign = (x >> 16) & 0x8000u;
        const uint32_t absx = x & 0x7fffffffu;
        if (absx > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
        if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // overflow to inf (incl. rounding)
        if (absx < 0x38800000u) {                                     // subnormal half or zero
            if (absx < 0x33000000u) return (uint16_t)sign;            // below half the smallest subnormal
            // value = mant * 2^(e-150); in units of 2^-24 that is mant >> (126 - e).
            const int e = (int)(absx >> 23);
            const uint32_t mant = (absx & 0x7fffffu) | 0x800000u;
            const int rshift = 126 - e;
            uint32_t r = mant >> rshift;
            const uint32_t rem = mant & ((1u << rshift) - 1u), half = 1u << (rshift - 1);
            if (rem > half || (rem == half && (r & 1u))) ++r;
            return (uint16_t)(sign | r);
        }
        uint32_t r = ((absx >> 13) - (112u << 10));
        const uint32_t rem = absx & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }

    float f16_to_f32(uint16_t h) {
        const int sign = h >> 15, exp = (h >> 10) & 31, man = h & 1023;
        float v;
        if (exp == 0) v = std::ldexp((float)man, -24);
        else if (exp == 31) v = man ? NAN : INFINITY;
        else v = std::ldexp((float)(man | 1024), exp - 25);
        return sign ? -v : v;
    }

    std::shared_ptr<Buffer> numpy_to_buffer(py::array array, DeviceEnum dev, std::optional<std::string> dtype_name) {
        const DType dt = dtype_name ? dtype_from_name(*dtype_name) : DType::Float32;
        std::vector<int> shape;
        for (py::ssize_t i = 0; i < array.ndim(); ++i) shape.push_back(checked_extent(array.shape(i), "Array dimension"));
        const size_t n = (size_t)array.size();
        std::vector<unsigned char> host;
        const void* src = nullptr;
        py::array keep;
        switch (dt) {
            case DType::Float32: {
                auto a = py::array_t<float, py::array::c_style | py::array::forcecast>::ensure(array);
                keep = a;
                src = a.data();
                break;
            }
            case DType::BFloat16: case DType::Float16: {
                auto a = py::array_t<float, py::array::c_style | py::array::forcecast>::ensure(array);
                host.resize(n * 2);
                uint16_t* h = (uint16_t*)host.data();
                for (size_t i = 0; i < n; ++i) h[i] = dt == DType::BFloat16 ? f32_to_bf16_rne(a.data()[i]) : f32_to_f16_rne(a.data()[i]);
                src = host.data();
                break;
            }
            case DType::Int64: {
                auto a = py::array_t<int64_t, py::array::c_style | py::array::forcecast>::ensure(array);
                keep = a;
                src = a.data();
                break;
            }
            case DType::Int32: {
                auto a = py::array_t<int32_t, py::array::c_style | py::array::forcecast>::ensure(array);
                keep = a;
                src = a.data();
                break;
            }
            case DType::Bool: {
                auto a = py::array_t<bool, py::array::c_style | py::array::forcecast>::ensure(array);
                keep = a;
                src = a.data();
                break;
            }
        }
        auto buf = empty(shape, dev, dt);
        if (buf->bytes) get_allocator(dev)->copy_host_to_device(buf->ptr, src, buf->bytes);
        return buf;
    }

    // Host copy of a buffer in its own element type; bf16/fp16 widen to float32.
    py::array buffer_to_numpy(const std::shared_ptr<Buffer>& buffer) {
        if (!buffer || (!buffer->ptr && buffer->bytes)) throw std::runtime_error("Cannot read from an empty or unrealized memory buffer.");
        IAllocator* alloc = get_allocator(buffer->device.type);
        std::vector<py::ssize_t> shape(buffer->shape.begin(), buffer->shape.end());
        auto copy_into = [&](void* dst) {
            if (buffer->bytes) alloc->copy_device_to_host(dst, buffer->ptr, buffer->bytes);
        };
        switch (buffer->dtype) {
            case DType::Float32: { py::array_t<float> r(shape); copy_into(r.mutable_data()); return r; }
            case DType::Int64: { py::array_t<int64_t> r(shape); copy_into(r.mutable_data()); return r; }
            case DType::Int32: { py::array_t<int32_t> r(shape); copy_into(r.mutable_data()); return r; }
            case DType::Bool: { py::array_t<bool> r(shape); copy_into(r.mutable_data()); return r; }
            case DType::BFloat16: case DType::Float16: {
                std::vector<uint16_t> h(buffer->numel());
                copy_into(h.data());
                py::array_t<float> r(shape);
                float* o = r.mutable_data();
                for (size_t i = 0; i < h.size(); ++i) o[i] = buffer->dtype == DType::BFloat16 ? bf16_to_f32(h[i]) : f16_to_f32(h[i]);
                return r;
            }
        }
        throw std::runtime_error("Unsupported DType.");
    }

    // Kernel planning without a launch (code generator tests on machines with
    // no GPU): the leaves' pointers are treated as opaque addresses.
    py::dict plan_kernel(const std::shared_ptr<Node>& root) {
        py::dict d;
        hip::KernelLaunch k;
        hip::ReducePlan rp;
        const int cu = 256;
        const std::shared_ptr<Node> red = ops::is_reduction(root->op) ? nullptr : hip::epilogue_reduction(root);
        if (red) {
            // An element-wise root that runs as a reduction's store epilogue:
            // the reduction's plan with the root's tape at its store. The
            // epilogue reads the reduction as a leaf, so it gets a host
            // stand-in buffer while the tape is built.
            const auto& x = red->parents[0];
            const hip::Expr e = hip::build_expr(x, x->view.shape, true);
            const auto& a = std::get<ReduceAttrs>(red->attrs);
            hip::StoreEpilogue ep;
            red->data = empty(red->view.shape, DeviceEnum::CPU, DType::Float32);
            try {
                ep.expr = hip::build_expr(root, root->view.shape, true);
            } catch (...) {
                red->data = nullptr;
                throw;
            }
            for (size_t L = 0; L < ep.expr.leaves.size(); ++L)
                if (ep.expr.leaves[L].ptr == red->data->ptr) ep.value = (int)L;
            red->data = nullptr;
            ep.out = (void*)(uintptr_t)0x200000;
            const hip::ReduceOp op = red->op == ops::OpEnum::SUM ? hip::ReduceOp::Sum : hip::ReduceOp::Max;
            rp = hip::plan_reduce(e, x->view.shape, a.axes, op, (void*)(uintptr_t)0x100000, cu, false, &ep);
            k = rp.first;
            d["two_pass"] = rp.two_pass;
            d["second_source"] = hip::kernel_source(rp.second);
            d["second_name"] = rp.second.name;
            d["workspace_bytes"] = rp.workspace_bytes;
            d["store_epilogue"] = true;
        } else if (ops::is_reduction(root->op)) {
            const auto& x = root->parents[0];
            const hip::Expr e = hip::build_expr(x, x->view.shape, true);
            const auto& a = std::get<ReduceAttrs>(root->attrs);
            const hip::ReduceOp op = root->op == ops::OpEnum::SUM ? hip::ReduceOp::Sum
                                     : root->op == ops::OpEnum::MAX ? hip::ReduceOp::Max : hip::ReduceOp::Argmax;
            rp = hip::plan_reduce(e, x->view.shape, a.axes, op, (void*)(uintptr_t)0x100000, cu);
            k = rp.first;
            d["two_pass"] = rp.two_pass;
            d["second_source"] = hip::kernel_source(rp.second);
            d["second_name"] = rp.second.name;
            d["workspace_bytes"] = rp.workspace_bytes;
        } else {
            const hip::Expr e = hip::build_expr(root, root->view.shape, true);
            k = hip::plan_map(e, root->view.shape, (void*)(uintptr_t)0x100000, root->dtype, cu);
            d["two_pass"] = false;
        }
        d["source"] = hip::kernel_source(k);
        d["name"] = k.name;
        d["plan"] = k.plan.text();
        d["grid"] = std::vector<uint32_t>{k.grid[0], k.grid[1], k.grid[2]};
        d["lds"] = k.lds;
        d["num_args"] = k.args.size();
        return d;
    }

    // The multi-output kernel realize_all would launch for these element-wise
    // roots of one shape (planning only: operands may live on any device).
    py::dict plan_group(const std::vector<std::shared_ptr<Node>>& roots) {
        if (roots.empty()) throw std::runtime_error("_plan_group: no roots");
        const auto& shape = roots[0]->view.shape;
        const hip::Expr e = hip::build_expr_multi(roots, shape, true);
        std::vector<void*> outs(roots.size(), (void*)(uintptr_t)0x100000);
        std::vector<DType> dts;
        for (const auto& r : roots) dts.push_back(r->dtype);
        const hip::KernelLaunch k = hip::plan_map_multi(e, shape, outs, dts, 256);
        py::dict d;
        d["source"] = hip::kernel_source(k);
        d["name"] = k.name;
        d["plan"] = k.plan.text();
        d["num_leaves"] = e.leaves.size();
        d["num_insts"] = e.insts.size();
        return d;
    }
}

PYBIND11_MODULE(ormi_backend, m) {
    m.doc() = "Ormi C++ backend with the MI355X (HIP) device";

    py::enum_<DeviceEnum>(m, "DeviceEnum")
        .value("CPU", DeviceEnum::CPU)
        .value("CUDA", DeviceEnum::CUDA)
        .value("HIP", DeviceEnum::HIP)
        .export_values();

    py::class_<Device>(m, "Device")
        .def(py::init<DeviceEnum, int>(), py::arg_v("type", DeviceEnum::CUDA, "DeviceEnum.CUDA"), py::arg("id") = 0)
        .def_readwrite("type", &Device::type)
        .def_readwrite("id", &Device::id)
        .def("__repr__", &Device::to_string)
        .def("is_type", [](const Device& d, const std::string& name) {
            if (name == "cuda" || name == "CUDA") return d.type == DeviceEnum::CUDA;
            if (name == "cpu" || name == "CPU") return d.type == DeviceEnum::CPU;
            if (name == "hip" || name == "HIP") return d.type == DeviceEnum::HIP;
            return false;
        });

    py::enum_<DType>(m, "DType")
        .value("Float32", DType::Float32).value("Int32", DType::Int32).value("Bool", DType::Bool)
        .value("BFloat16", DType::BFloat16).value("Float16", DType::Float16).value("Int64", DType::Int64)
        .export_values();

    {
        auto e = py::enum_<ops::OpEnum>(m, "OpEnum");
        for (int i = (int)ops::OpEnum::LEAF; i <= (int)ops::OpEnum::CAST; ++i) {
            auto op = (ops::OpEnum)i;
            e.value(ops::op_name(op), op);
        }
        e.export_values();
    }

    py::class_<Buffer, std::shared_ptr<Buffer>>(m, "DataBuffer")
        .def_property_readonly("bytes", [](const Buffer& b) { return b.bytes; })
        .def_property_readonly("shape", [](const Buffer& b) { return b.shape; })
        .def_property_readonly("dtype", [](const Buffer& b) { return std::string(dtype_name(b.dtype)); })
        .def_property_readonly("device", [](const Buffer& b) { return b.device; })
        .def_property_readonly("ptr", [](const Buffer& b) { return (uintptr_t)b.ptr; })
        .def("__str__", [](const Buffer& b) { return to_string(b); });

    m.def("numpy_to_buffer", &numpy_to_buffer, py::arg("array"), py::arg("device"), py::arg("dtype") = std::nullopt);
    m.def("buffer_to_numpy", &buffer_to_numpy);

    py::class_<TensorView>(m, "TensorView")
        .def(py::init<>())
        .def(py::init([](std::vector<int> shape, std::vector<int> strides) {
            if (shape.size() != strides.size()) throw std::runtime_error("TensorView: shape and strides differ in length.");
            TensorView v;
            v.shape = std::move(shape);
            v.strides = std::move(strides);
            return v;
        }))
        .def_readwrite("shape", &TensorView::shape)
        .def_readwrite("strides", &TensorView::strides)
        .def("is_contiguous", &TensorView::is_contiguous);

    py::class_<Node, std::shared_ptr<Node>>(m, "Node")
        .def(py::init<std::shared_ptr<Buffer>, bool, Device>())
        .def(py::init([](ops::OpEnum op, std::vector<std::shared_ptr<Node>> parents, Device dev) {
            return std::make_shared<Node>(op, std::move(parents), dev);
        }))
        .def_property_readonly("op", [](const Node& n) { return n.op; })
        .def_property_readonly("requires_grad", [](const Node& n) { return n.requires_grad; })
        .def_property_readonly("is_realized", &Node::is_realized)
        .def_property_readonly("shape", [](const Node& n) { return n.view.shape; })
        .def_property_readonly("strides", [](const Node& n) { return n.view.strides; })
        .def_property_readonly("dtype", [](const Node& n) { return std::string(dtype_name(n.dtype)); })
        .def_property_readonly("parents", [](const Node& n) { return n.parents; })
        .def_property_readonly("device", [](const Node& n) { return n.device; })
        .def_property_readonly("axes", [](const Node& n) {
            if (auto r = std::get_if<ReduceAttrs>(&n.attrs)) return r->axes;
            if (auto p = std::get_if<PermuteAttrs>(&n.attrs)) return p->axes;
            return std::vector<int>{};
        })
        .def_property_readonly("keepdims", [](const Node& n) {
            auto r = std::get_if<ReduceAttrs>(&n.attrs);
            return r ? r->keepdims : false;
        })
        .def_readwrite("view", &Node::view)
        .def_readwrite("data", &Node::data)
        .def_readwrite("grad", &Node::grad)
        // node.grad = None through the property costs a failed holder
        // conversion first (about 0.7 us); Tensor.zero_grad calls this instead.
        .def("_clear_grad", [](Node& n) { n.grad.reset(); });

    // Internal fast paths for ormi_amd.Tensor's operators: two node arguments
    // instead of a list, the device taken from the first operand.
    m.def("_binary", &ops::binary);
    m.def("_unary", &ops::unary);
    m.def("add", &ops::add);
    m.def("sub", &ops::sub);
    m.def("mul", &ops::mul);
    m.def("div", &ops::div);
    m.def("pow", &ops::pow);
    m.def("eq", &ops::eq);
    m.def("neg", &ops::neg);
    m.def("exp", &ops::exp);
    m.def("log", &ops::log);
    m.def("sin", &ops::sin);
    m.def("cos", &ops::cos);
    m.def("relu", &ops::relu);
    m.def("step", &ops::step);
    m.def("tanh", &ops::tanh);
    m.def("sigmoid", &ops::sigmoid);
    m.def("gelu", &ops::gelu);
    m.def("matmul", &ops::matmul);
    m.def("sum", &ops::sum, py::arg("node"), py::arg("axes"), py::arg("keepdims") = false);
    m.def("max", &ops::max, py::arg("node"), py::arg("axes"), py::arg("keepdims") = false);
    m.def("argmax", &ops::argmax, py::arg("node"), py::arg("axes"), py::arg("keepdims") = false);
    m.def("transpose", &ops::transpose);
    m.def("expand", &ops::expand);
    m.def("reshape", &ops::reshape);
    m.def("cast", [](std::shared_ptr<Node> x, const std::string& dt) { return ops::cast(x, dtype_from_name(dt)); });

    m.def("execute_graph", &execute_graph);
    // Run the device's element-wise JIT on root with whatever tape reaches it
    // (the reference's cpu::execute_jit / cuda::execute_jit entry).
    m.def("execute_jit", [](std::shared_ptr<Node> root) { run_jit(root); });
    m.def("calc_contiguous_strides", &calc_contiguous_strides);
    m.def("broadcast_shapes", &broadcast_shapes);
    m.def("execute_graph_eager", &execute_graph_eager);
    m.def("compute_gradients", &compute_gradients);
    m.def("zero_grad_graph", &zero_grad_graph);

    m.def("has_allocator", [](DeviceEnum d) { return has_allocator(d); });
    m.def("hip_available", [] {
        try {
            get_allocator(DeviceEnum::HIP);
            return true;
        } catch (const std::exception&) {
            return false;
        }
    });
    m.def("synchronize", [] { ORMI_HIP_CHECK(ormi_hip_synchronize()); });
    m.def("_size_class", &hip::size_class);
    m.def("allocator_stats", [] {
        const hip::AllocatorStats st = hip::allocator_stats();
        py::dict d;
        d["live_bytes"] = st.live_bytes;
        d["cached_bytes"] = st.cached_bytes;
        d["device_bytes"] = st.device_bytes;
        d["device_mallocs"] = st.device_mallocs;
        d["device_frees"] = st.device_frees;
        d["reuses"] = st.reuses;
        return d;
    }, "HIP caching allocator counters.");
    m.def("empty_cache", &hip::empty_cache, "Return every cached HIP block to the device.");
    m.def("gemm_epilogue_count", &hip::gemm_epilogue_count,
          "Element-wise nodes realized as a GEMM epilogue (ormi_hip_gemm_ex) in this process.");
    m.def("set_gemm_epilogue", &hip::set_gemm_epilogue, py::arg("on"),
          "Turn GEMM epilogue fusion on or off (default: on unless ORMI_GEMM_EPILOGUE=0).");
    m.def("gemm_pair_count", &hip::gemm_pair_count,
          "Pairs of independent products the HIP scheduler ran as one grouped GEMM launch in this process.");
    m.def("_plan_kernel", &plan_kernel);
    m.def("_plan_group", &plan_group);
    m.def("realize_all", &execute_graph_group,
          "Realize several nodes together; on the HIP device same-shape element-wise roots share one kernel.");
    m.def("_fastdiv", [](uint32_t d) {
        auto f = hip::make_fastdiv(d);
        return py::make_tuple(f.m, f.s);
    });
    m.def("_rtc_options", [] { return hip::rtc_options(); });
    m.def("_is_store_epilogue", [](const std::shared_ptr<Node>& n) { return hip::epilogue_reduction(n) != nullptr; },
          "Whether the element-wise region of n would run as a reduction's store epilogue.");
    m.def("_kernel_launches", [] { return hip::kernel_launches(); },
          "Generated (hipRTC) kernels launched by this process so far.");
}
