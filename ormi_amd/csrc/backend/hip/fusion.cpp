// Pointwise region discovery and the SSA tape the code generator consumes.
// Follows the reference's tape construction (csrc/backend/cuda/compiler.cu:22-51:
// dedup by Node*, realized nodes become leaves, MATMUL is never fused) but
// walks the whole unrealized pointwise region instead of a single op, and
// aligns each leaf to the kernel's shape the way the reference's CPU JIT
// does (csrc/backend/cpu/jit.cpp:24-46: right-aligned, size-1 dims and
// 1-element buffers read with stride 0).
#include <mutex>
#include <unordered_map>
#include <unordered_set>

#include "backend/hip/hip_backend.h"
#include "backend/hip/small_containers.h"
#include "runtime/runtime.h"

namespace ormi::hip {
    using ops::OpEnum;

    static std::unordered_map<OpEnum, LoweringFunc>& lowering_table() {
        static std::unordered_map<OpEnum, LoweringFunc> t;
        return t;
    }

    // The registered function per op, indexed by the op's value: the graph
    // walks ask for every node they visit. unordered_map elements keep their
    // addresses across inserts, so the pointers stay valid.
    constexpr size_t kOpSlots = 64;
    static_assert((size_t)OpEnum::CAST < kOpSlots, "op table too small");
    static const LoweringFunc* lowering_slots[kOpSlots] = {};

    void HIPLoweringRegistry::register_func(OpEnum op, LoweringFunc f) {
        LoweringFunc& slot = lowering_table()[op];
        slot = std::move(f);
        lowering_slots[(size_t)op] = &slot;
    }
    bool HIPLoweringRegistry::has(OpEnum op) { return find(op) != nullptr; }
    const LoweringFunc* HIPLoweringRegistry::find(OpEnum op) {
        const size_t i = (size_t)op;
        return i < kOpSlots ? lowering_slots[i] : nullptr;
    }
    LoweringFunc HIPLoweringRegistry::get(OpEnum op) {
        auto it = lowering_table().find(op);
        if (it == lowering_table().end())
            throw std::runtime_error(std::string("HIP JIT Compiler Error: No lowering rule registered for ") + ops::op_name(op));
        return it->second;
    }

    namespace {
        // The built-in lowerings go into the registry at load time; a backend
        // extension may register more (or replace one) afterwards.
        struct RegisterBuiltins {
            RegisterBuiltins() {
                for (OpEnum op : {OpEnum::ADD, OpEnum::SUB, OpEnum::MUL, OpEnum::DIV, OpEnum::POW, OpEnum::EQ, OpEnum::NEG,
                                  OpEnum::EXP, OpEnum::LOG, OpEnum::SIN, OpEnum::COS, OpEnum::RELU, OpEnum::STEP,
                                  OpEnum::TANH, OpEnum::TANH_GRAD, OpEnum::SIGMOID, OpEnum::SIGMOID_GRAD, OpEnum::GELU,
                                  OpEnum::GELU_GRAD})
                    HIPLoweringRegistry::register_func(op, *builtin_lowering(op));
            }
        } register_builtins;
    }

    static bool cast_target_is_float(const Node& n) {
        const DType t = std::get<CastAttrs>(n.attrs).dtype;
        return t == DType::Float32 || t == DType::BFloat16 || t == DType::Float16;
    }

    bool fusible_root(const Node& n) {
        if (n.is_realized() || !ops::is_pointwise(n.op)) return false;
        return n.op == OpEnum::CAST || HIPLoweringRegistry::has(n.op);
    }

    bool fusible_interior(const Node& n) {
        if (!fusible_root(n)) return false;
        return n.op != OpEnum::CAST || cast_target_is_float(n);
    }

    size_t region_size(const NodePtr& root, size_t limit);

    // A scalar seen through views: n is an unrealized view (a broadcast, a
    // reshape, ...) whose source, down its chain of unrealized views, is an
    // unrealized element-wise node of ONE element with a region of at most
    // kMaxScalarRegion ops. Every element of n is that scalar, and its region
    // reads only one-element operands (an element-wise op does not reduce), which
    // a kernel of any shape reads with stride 0: so a consumer's kernel
    // evaluates it itself instead of realizing it first, a kernel of one
    // element (the loss's seed times its scale in a backward pass, before the
    // broadcast to the loss's input). Returns the source, or nullptr.
    constexpr size_t kMaxScalarRegion = 16;
    static const NodePtr* scalar_view_source(const NodePtr& n) {
        if (n->is_realized() || !is_view_op(n->op) || n->parents.empty()) return nullptr;
        const NodePtr* src = &n->parents[0];
        while (!(*src)->is_realized() && is_view_op((*src)->op) && !(*src)->parents.empty()) src = &(*src)->parents[0];
        const Node& s = **src;
        if (s.is_realized() || !fusible_interior(s) || shape_numel(s.view.shape) != 1) return nullptr;
        return region_size(*src, kMaxScalarRegion) <= kMaxScalarRegion ? src : nullptr;
    }

    std::vector<NodePtr> region_frontier(const NodePtr& root) {
        std::vector<NodePtr> frontier;
        SmallSet<Node> seen;
        seen.insert(root.get());
        SmallVec<Node*, 64> stack;
        stack.push_back(root.get());
        size_t interior = 1;
        while (!stack.empty()) {
            Node* n = stack.back();
            stack.pop_back();
            for (const auto& p : n->parents) {
                if (!seen.insert(p.get())) continue;
                if (p->is_realized()) continue;
                // Past kMaxRegion interior nodes, element-wise nodes become frontier:
                // they are realized first, as regions of their own.
                if (fusible_interior(*p) && interior < kMaxRegion) {
                    stack.push_back(p.get());
                    ++interior;
                } else if (const NodePtr* src = interior < kMaxRegion ? scalar_view_source(p) : nullptr) {
                    if (seen.insert(src->get())) {
                        stack.push_back(src->get());
                        ++interior;
                    }
                } else {
                    frontier.push_back(p);
                }
            }
        }
        return frontier;
    }

    size_t region_size(const NodePtr& root, size_t limit) {
        if (root->is_realized() || !fusible_root(*root)) return 0;
        SmallSet<Node> seen;
        seen.insert(root.get());
        SmallVec<Node*, 64> stack;
        stack.push_back(root.get());
        size_t interior = 1;
        while (!stack.empty() && interior <= limit) {
            Node* n = stack.back();
            stack.pop_back();
            for (const auto& p : n->parents) {
                if (!seen.insert(p.get()) || p->is_realized()) continue;
                Node* q = p.get();
                if (!fusible_interior(*p)) {
                    // A scalar seen through views counts with its own region
                    // (whose size the source check bounds).
                    const NodePtr* src = limit > kMaxScalarRegion ? scalar_view_source(p) : nullptr;
                    if (!src || !seen.insert(src->get())) continue;
                    q = src->get();
                }
                stack.push_back(q);
                ++interior;
            }
        }
        return interior;
    }

    static Leaf make_leaf(const NodePtr& n, const std::vector<int>& shape, bool plan_only) {
        if (!n->data) throw std::runtime_error("HIP codegen: leaf is not realized.");
        if (!plan_only && n->device.type != DeviceEnum::HIP) throw std::runtime_error("HIP codegen: operand lives on another device.");
        Leaf L;
        L.keep = n;
        L.ptr = n->data->ptr;
        L.dtype = n->data->dtype;
        const size_t ndim = shape.size();
        L.st.assign(ndim, 0);
        // Scalar rule of the reference (csrc/backend/cpu/jit.cpp:24): a leaf whose
        // view is 0-d or whose buffer holds one element reads element 0.
        L.scalar = n->view.shape.empty() || n->data->numel() == 1;
        if (L.scalar) return L;
        const auto& ls = n->view.shape;
        const auto& lst = n->view.strides;
        if (ls.size() > ndim) throw std::runtime_error("HIP codegen: operand has more dims than the kernel shape.");
        const size_t off = ndim - ls.size();
        for (size_t d = off; d < ndim; ++d) {
            const int od = (int)(d - off);
            if (ls[od] != 1) {
                if (ls[od] != shape[d]) throw std::runtime_error("HIP codegen: operand shape does not broadcast to the kernel shape.");
                L.st[d] = lst[od];
            }
        }
        return L;
    }

    Expr build_expr(const NodePtr& root, const std::vector<int>& shape, bool plan_only) {
        return build_expr_multi({root}, shape, plan_only);
    }

    Expr build_expr_multi(const std::vector<NodePtr>& roots, const std::vector<int>& shape, bool plan_only) {
        Expr e;
        e.leaves.reserve(8);
        e.roots.reserve(roots.size());
        SmallMap<Node, int> value_of;
        SmallSet<Node, 8> root_set;
        for (const auto& r : roots) root_set.insert(r.get());
        // Post-order DFS over the union of the roots' regions: leaves get ids as
        // first seen, interior nodes after all their operands. A node shared by
        // several roots (or a root inside another root's region) is one value.
        struct Frame { Node* n; size_t next; };
        SmallVec<Frame, 64> stack;
        auto is_interior = [&](const Node* n) {
            return root_set.contains(n) ? fusible_root(*n) : fusible_interior(*n);
        };
        auto visit_leaf = [&](const NodePtr& n) {
            const int id = (int)e.leaves.size();
            e.leaves.push_back(make_leaf(n, shape, plan_only));
            value_of.insert(n.get(), id);
        };
        if (roots.size() == 1 && !is_interior(roots[0].get())) {
            // A realized node (or a reduction input that is already a buffer):
            // the tape is the identity on one leaf.
            visit_leaf(roots[0]);
            e.root = 0;
            e.roots = {0};
            return e;
        }
        SmallVec<Node*, 64> interior_post;
        SmallSet<Node> on_stack;
        // Views read as the scalar they broadcast: the view's value is its source's.
        SmallMap<Node, Node*> through;
        for (const auto& root : roots) {
            if (!is_interior(root.get())) throw std::runtime_error("HIP codegen: a grouped root is not an element-wise node.");
            if (value_of.find(root.get())) continue;  // inside an earlier root's region
            on_stack.insert(root.get());
            stack.push_back({root.get(), 0});
            while (!stack.empty()) {
                Frame& f = stack.back();
                if (f.next < f.n->parents.size()) {
                    const NodePtr& p = f.n->parents[f.next++];
                    if (value_of.find(p.get()) || on_stack.contains(p.get()) || through.find(p.get())) continue;
                    if (!p->is_realized() && is_interior(p.get())) {
                        on_stack.insert(p.get());
                        stack.push_back({p.get(), 0});
                    } else if (const NodePtr* src = scalar_view_source(p)) {
                        through.insert(p.get(), src->get());
                        Node* q = src->get();
                        if (!value_of.find(q) && !on_stack.contains(q)) {
                            on_stack.insert(q);
                            stack.push_back({q, 0});
                        }
                    } else {
                        if (!p->is_realized()) throw std::runtime_error("HIP codegen: region input was not realized first.");
                        visit_leaf(p);
                    }
                } else {
                    Node* n = f.n;
                    interior_post.push_back(n);
                    value_of.insert(n, -1);  // assigned below
                    on_stack.erase(n);
                    stack.pop_back();
                }
            }
        }
        const int nleaves = (int)e.leaves.size();
        for (size_t k = 0; k < interior_post.size(); ++k) value_of.set(interior_post[k], nleaves + (int)k);
        auto id_of = [&](const Node* n) {
            if (Node* const* q = through.find(n)) n = *q;
            const int* v = value_of.find(n);
            if (!v) throw std::runtime_error("HIP codegen: operand without a value.");
            return *v;
        };
        e.insts.reserve(interior_post.size());
        for (size_t k = 0; k < interior_post.size(); ++k) {
            const Node* n = interior_post[k];
            Inst in;
            in.op = n->op;
            in.a = id_of(n->parents[0].get());
            if (ops::op_arity(n->op) == 2) in.b = id_of(n->parents[1].get());
            if (n->op == OpEnum::CAST) in.cast = std::get<CastAttrs>(n->attrs).dtype;
            else in.lower = HIPLoweringRegistry::find(n->op);
            e.insts.push_back(in);
        }
        for (const auto& r : roots) e.roots.push_back(id_of(r.get()));
        e.root = e.roots[0];
        return e;
    }
}
