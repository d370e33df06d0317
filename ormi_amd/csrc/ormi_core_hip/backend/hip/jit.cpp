// hip::execute_jit: the HIP case of execute_graph (csrc/backend/runtime.cpp:
// 29-38), in place of cuda::execute_jit (csrc/backend/cuda/jit.cu:13-44).
//
// The walk is the reference's tape (csrc/backend/cuda/compiler.cu:22-51):
// every node is visited once (dedup by Node*), a realized node is a leaf, any
// other node one instruction over earlier values, and MATMUL cannot be part of
// an element-wise tape. Instead of NVRTC source, the tape goes to
// ormi_hip_map as an ormi_map_desc; libormi_hip generates one gfx950 kernel
// for its structure, caches it, and launches it on its stream (replacing
// compile_ptx, the module load, cuLaunchKernel and the unload, jit.cu:21-43).
//
// Leaf layout follows the reference exactly (compiler.cu:76-101, and its CPU
// twin csrc/backend/cpu/jit.cpp:22-46): a leaf whose view has no dims or whose
// buffer holds one float is a scalar; otherwise its dims align to the output's
// from the right, and a dim of extent 1 (or one the leaf lacks) gets stride 0.
// The output is a new contiguous buffer of the root's shape (jit.cu:26-28).
#include <unordered_map>
#include <utility>
#include <vector>

#include "backend/hip/hip_safe_call.h"
#include "backend/hip/jit.h"
#include "core/memory.h"
#include "core/shape.h"

namespace ormi::hip {
    namespace {
        int map_op(ops::OpEnum op) {
            switch (op) {
                case ops::OpEnum::NEG: return ORMI_MAP_NEG;
                case ops::OpEnum::EXP: return ORMI_MAP_EXP;
                case ops::OpEnum::LOG: return ORMI_MAP_LOG;
                case ops::OpEnum::SIN: return ORMI_MAP_SIN;
                case ops::OpEnum::COS: return ORMI_MAP_COS;
                case ops::OpEnum::ADD: return ORMI_MAP_ADD;
                case ops::OpEnum::SUB: return ORMI_MAP_SUB;
                case ops::OpEnum::MUL: return ORMI_MAP_MUL;
                case ops::OpEnum::DIV: return ORMI_MAP_DIV;
                case ops::OpEnum::POW: return ORMI_MAP_POW;
                case ops::OpEnum::MATMUL:
                    throw std::runtime_error("FATAL: MATMUL cannot be fused into a 1D element-wise kernel.");
                default:
                    throw std::runtime_error("HIP JIT: op has no element-wise lowering.");
            }
        }

        bool is_binary(int op) { return op >= ORMI_MAP_ADD && op <= ORMI_MAP_POW; }

        // The tape of `root`: leaves in first-visit order, instructions in
        // post-order, operands as references (k >= 0: instruction k, -1 - i:
        // leaf i). Returns the root's reference.
        int build_tape(const std::shared_ptr<Node>& root, const std::vector<int>& out_shape,
                       std::vector<ormi_map_leaf>& leaves, std::vector<ormi_map_inst>& insts) {
            const int nd = (int)out_shape.size();
            std::unordered_map<const Node*, int> ref;
            // (node, next parent to visit)
            std::vector<std::pair<Node*, size_t>> stack{{root.get(), 0}};
            while (!stack.empty()) {
                auto& [n, next] = stack.back();
                if (ref.count(n)) {
                    stack.pop_back();
                    continue;
                }
                if (n->is_realized()) {
                    ormi_map_leaf L{};
                    L.ptr = n->data->ptr;
                    L.dtype = ORMI_DTYPE_F32;
                    L.scalar = n->view.shape.empty() || n->data->bytes / sizeof(float) == 1;
                    if (!L.scalar) {
                        const int off = nd - (int)n->view.shape.size();
                        if (off < 0) throw std::runtime_error("HIP JIT: a leaf has more dims than the output.");
                        for (int d = 0; d < nd; ++d) {
                            const int od = d - off;
                            L.strides[d] = (od >= 0 && n->view.shape[od] != 1) ? n->view.strides[od] : 0;
                        }
                    }
                    leaves.push_back(L);
                    ref[n] = -(int)leaves.size();
                    stack.pop_back();
                    continue;
                }
                if (next < n->parents.size()) {
                    Node* p = n->parents[next++].get();
                    if (!ref.count(p)) stack.emplace_back(p, 0);
                    continue;
                }
                const int op = map_op(n->op);
                const size_t arity = is_binary(op) ? 2 : 1;
                if (n->parents.size() != arity) throw std::runtime_error("HIP JIT: wrong number of operands.");
                ormi_map_inst in{};
                in.op = op;
                in.a = ref.at(n->parents[0].get());
                in.b = arity == 2 ? ref.at(n->parents[1].get()) : 0;
                insts.push_back(in);
                ref[n] = (int)insts.size() - 1;
                stack.pop_back();
            }
            return ref.at(root.get());
        }
    }

    void execute_jit(std::shared_ptr<Node> root) {
        const std::vector<int> out_shape = root->view.shape;
        if ((int)out_shape.size() > ORMI_MAP_MAX_DIMS) throw std::runtime_error("HIP JIT: more than 8 dims.");
        std::vector<ormi_map_leaf> leaves;
        std::vector<ormi_map_inst> insts;
        const int root_ref = build_tape(root, out_shape, leaves, insts);

        // ormi_map_desc numbers the leaves first, then the instructions.
        const int nl = (int)leaves.size();
        auto value = [nl](int r) { return r < 0 ? -1 - r : nl + r; };
        for (auto& in : insts) {
            in.a = value(in.a);
            if (is_binary(in.op)) in.b = value(in.b);
        }

        root->data = empty(out_shape, DeviceEnum::HIP);
        root->view.shape = out_shape;
        root->view.strides = calc_contiguous_strides(out_shape);

        ormi_map_desc d{};
        d.ndim = (int)out_shape.size();
        for (int i = 0; i < d.ndim; ++i) d.shape[i] = out_shape[i];
        d.num_leaves = nl;
        d.leaves = leaves.data();
        d.num_insts = (int)insts.size();
        d.insts = insts.data();
        int out_value = value(root_ref);
        int out_dtype = ORMI_DTYPE_F32;
        void* out = root->data->ptr;
        d.num_outputs = 1;
        d.output_values = &out_value;
        d.outputs = &out;
        d.output_dtypes = &out_dtype;
        HIP_SAFE_CALL(ormi_hip_map(&d));
    }
}
