// HIP device: fusion scheduler and graph breakers (the allocator is in
// allocator.cpp).
//
// Scheduler: the reference realizes every parent before compiling a node
// (csrc/backend/runtime.cpp:16-18), so each op is its own kernel and every
// intermediate round-trips through HBM. On the HIP device, realize(root):
//   * view        -> realize the parent, alias its buffer (runtime.cpp:20-23);
//   * pointwise   -> realize only the region's frontier (views, reductions,
//                    matmuls, realized nodes), then ONE fused kernel writes
//                    root; interior pointwise nodes stay unrealized and are
//                    recomputed by any later kernel that reads them;
//   * SUM/MAX/ARGMAX -> the producing pointwise region is fused into the
//                    reduction as its prologue;
//   * MATMUL      -> both operands realized, MFMA GEMM.
// Reductions and MATMUL are registered as graph breakers for DeviceEnum::HIP
// (the reference's plugin point, csrc/backend/graph_breakers.h:12-14).
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "backend/hip/hip_backend.h"
#include "backend/hip/small_containers.h"
#include "core/allocator.h"
#include "core/memory.h"
#include "runtime/graph_breakers.h"
#include "runtime/runtime.h"

namespace ormi::hip {
    using ops::OpEnum;

    int device_compute_units() {
        static int cu = [] {
            ormi_hip_props p{};
            return ormi_hip_get_props(&p) == ORMI_HIP_OK && p.compute_units > 0 ? p.compute_units : 256;
        }();
        return cu;
    }

    // Realize what a reduction reads: a pointwise producer of at most
    // kMaxPrologue ops stays unrealized (it becomes the prologue); anything
    // else is realized.
    static bool fuse_as_prologue(const NodePtr& x) {
        return !x->is_realized() && fusible_root(*x) && region_size(x, kMaxPrologue) <= kMaxPrologue;
    }

    static void prepare_input(const NodePtr& x) {
        if (x->is_realized()) return;
        if (fuse_as_prologue(x)) {
            for (const auto& f : region_frontier(x)) realize(f);
        } else {
            realize(x);
        }
    }

    static void run_map(const NodePtr& root);

    // Element-wise regions of at most this many ops run as a reduction's store
    // epilogue (the mean is one multiply).
    constexpr size_t kMaxStoreEpilogue = 16;

    // The reduction whose store epilogue region `n` can be: n is an unrealized
    // fp32 element-wise root whose region reads exactly one unrealized node,
    // a SUM or MAX with n's own shape, besides realized scalars (1-element
    // buffers, such as the mean's 1/N). The region then costs no kernel and no
    // pass over the reduction's result. nullptr when the region is not of that
    // form.
    NodePtr epilogue_reduction(const NodePtr& n) {
        if (n->is_realized() || n->dtype != DType::Float32 || !fusible_root(*n)) return nullptr;
        NodePtr red;
        SmallSet<Node> seen;
        seen.insert(n.get());
        SmallVec<Node*, 16> stack;
        stack.push_back(n.get());
        size_t interior = 1;
        while (!stack.empty()) {
            Node* m = stack.back();
            stack.pop_back();
            for (const auto& p : m->parents) {
                if (!seen.insert(p.get())) continue;
                if (p->is_realized()) {
                    if (p->data->numel() != 1) return nullptr;
                    continue;
                }
                if (fusible_interior(*p)) {
                    if (++interior > kMaxStoreEpilogue) return nullptr;
                    stack.push_back(p.get());
                    continue;
                }
                if (red || (p->op != OpEnum::SUM && p->op != OpEnum::MAX) || p->dtype != DType::Float32 ||
                    p->view.shape != n->view.shape)
                    return nullptr;
                red = p;
            }
        }
        return red;
    }

    // The reduction `root`. With `epi`, an element-wise consumer of root's
    // result (epilogue_reduction(epi) == root) is realized by the same kernel:
    // it runs as the reduction's store epilogue and root's own result is
    // stored as well, so both nodes hold buffers afterwards.
    static void reduce_handler(const NodePtr& root, ReduceOp op, const NodePtr& epi = nullptr) {
        const NodePtr& x = root->parents[0];
        prepare_input(x);
        const auto& attrs = std::get<ReduceAttrs>(root->attrs);
        const std::vector<int>& in_shape = x->view.shape;
        const long long in_numel = shape_numel(in_shape);
        const DType out_dtype = op == ReduceOp::Argmax ? DType::Int64 : DType::Float32;
        auto out = empty(root->view.shape, DeviceEnum::HIP, out_dtype);
        root->data = out;
        root->view.strides = calc_contiguous_strides(root->view.shape);
        if (out->numel() == 0 || in_numel == 0) {
            if (out->numel() > 0) {
                if (op != ReduceOp::Sum) throw std::runtime_error("zero-size array to reduction operation maximum which has no identity");
                const float zero = 0.0f;
                ORMI_HIP_CHECK(ormi_hip_fill(out->ptr, &zero, 4, out->numel()));
            }
            if (epi) run_map(epi);  // root holds its buffer now: a plain element-wise kernel
            return;
        }
        const Expr e = build_expr(x, in_shape);
        StoreEpilogue ep;
        std::shared_ptr<Buffer> epi_out;
        if (epi) {
            // root is realized now, so the consumer's tape reads it as a leaf.
            ep.expr = build_expr(epi, epi->view.shape);
            for (size_t L = 0; L < ep.expr.leaves.size(); ++L)
                if (ep.expr.leaves[L].ptr == out->ptr) ep.value = (int)L;
            epi_out = empty(epi->view.shape, DeviceEnum::HIP, epi->dtype);
            ep.out = epi_out->ptr;
            ep.out_dtype = epi->dtype;
        }
        ReducePlan plan = plan_reduce(e, in_shape, attrs.axes, op, out->ptr, device_compute_units(), true, epi ? &ep : nullptr);
        if (epi) {
            epi->data = epi_out;
            epi->view.strides = calc_contiguous_strides(epi->view.shape);
        }
        std::shared_ptr<Buffer> ws;
        if (plan.two_pass) {
            ws = empty({(int)((plan.workspace_bytes + 3) / 4)}, DeviceEnum::HIP, DType::Float32);
            bind_workspace(plan, ws->ptr);
        }
        launch(plan.first);
        if (plan.two_pass) launch(plan.second);
        // ws returns to the pool here; later work on the same stream is ordered
        // after these kernels, so reuse is safe.
    }

    // Operand of a GEMM in the form ormi_hip_gemm takes: dtype f32/bf16/f16,
    // realized. Other dtypes (and mixed pairs) are converted to f32 by a fused
    // cast kernel.
    static NodePtr gemm_operand(const NodePtr& x, DType want) {
        realize(x);
        if (x->data->dtype == want) return x;
        auto c = std::make_shared<Node>(OpEnum::CAST, std::vector<NodePtr>{x}, x->device, CastAttrs{want});
        realize(c);
        return c;
    }

    // The descriptor of MATMUL node `root`'s product into `out` (contiguous
    // fp32, root's shape): same shape rule as the reference, trans/ld derived
    // from strides, batch dims broadcast with stride 0. Realizes the operands
    // (converting other dtypes); `hold` keeps the nodes whose buffers the
    // descriptor points at.
    static ormi_gemm_desc gemm_desc(const NodePtr& root, float* out, std::vector<NodePtr>& hold) {
        NodePtr A = root->parents[0], B = root->parents[1];
        realize(A);
        realize(B);
        DType dt = A->data->dtype;
        const bool same_float = dt == B->data->dtype && (dt == DType::Float32 || dt == DType::BFloat16 || dt == DType::Float16);
        if (!same_float) dt = DType::Float32;
        A = gemm_operand(A, dt);
        B = gemm_operand(B, dt);

        const auto& va = A->view;
        const auto& vb = B->view;
        const auto& vo = root->view;
        const int na = (int)va.shape.size(), nb = (int)vb.shape.size(), no = (int)vo.shape.size();

        ormi_gemm_desc d{};
        d.dtype = dt == DType::Float32 ? ORMI_DTYPE_F32 : dt == DType::BFloat16 ? ORMI_DTYPE_BF16 : ORMI_DTYPE_F16;
        d.M = va.shape[na - 2];
        d.K = va.shape[na - 1];
        d.N = vb.shape[nb - 1];
        d.a = A->data->ptr;
        d.a_stride_m = va.strides[na - 2];
        d.a_stride_k = va.strides[na - 1];
        d.b = B->data->ptr;
        d.b_stride_k = vb.strides[nb - 2];
        d.b_stride_n = vb.strides[nb - 1];
        d.c = out;
        // Batch dims: drop extent-1 dims, then each operand's batch stride is its
        // own stride where it has that dim with extent > 1, else 0 (broadcast).
        std::vector<int> bshape;
        std::vector<long long> abs, bbs;
        for (int i = 0; i < no - 2; ++i) {
            if (vo.shape[i] == 1) continue;
            auto stride_of = [&](const TensorView& v, int nd) -> long long {
                const int td = i - ((no - 2) - (nd - 2));
                return (td >= 0 && v.shape[td] > 1) ? v.strides[td] : 0;
            };
            bshape.push_back(vo.shape[i]);
            abs.push_back(stride_of(va, na));
            bbs.push_back(stride_of(vb, nb));
        }
        // Merge batch dims while both operands stay linear (keeps within 4 dims).
        for (size_t i = 0; i + 1 < bshape.size();) {
            if (abs[i] == abs[i + 1] * bshape[i + 1] && bbs[i] == bbs[i + 1] * bshape[i + 1]) {
                bshape[i] *= bshape[i + 1];
                abs[i] = abs[i + 1];
                bbs[i] = bbs[i + 1];
                bshape.erase(bshape.begin() + i + 1);
                abs.erase(abs.begin() + i + 1);
                bbs.erase(bbs.begin() + i + 1);
            } else {
                ++i;
            }
        }
        if (bshape.size() > ORMI_GEMM_MAX_BATCH_DIMS) throw std::runtime_error("HIP MATMUL: more than 4 non-mergeable batch dims.");
        d.batch_ndim = (int)bshape.size();
        for (size_t i = 0; i < bshape.size(); ++i) {
            d.batch_shape[i] = bshape[i];
            d.a_batch_stride[i] = abs[i];
            d.b_batch_stride[i] = bbs[i];
        }
        hold.push_back(A);
        hold.push_back(B);
        return d;
    }

    // A GEMM ready to launch: node n gets `out` once it has run (and the
    // product node g gets `aux`, for an activation epilogue). n is the MATMUL
    // itself for a plain product, else the element-wise node its epilogue
    // computes.
    struct PreparedGemm {
        NodePtr n, g;
        ormi_gemm_desc d{};
        ormi_gemm_epilogue e{};
        std::shared_ptr<Buffer> out, aux;
        std::vector<NodePtr> hold;
        bool empty = false;  // no elements: nothing to launch
    };

    static void commit(PreparedGemm& p);
    static bool launch_paired(PreparedGemm& self);

    // MATMUL on the HIP device (replaces cuda::matmul, csrc/backend/cuda/kernels/blas/
    // matmul.cu:19-122).
    static void prepare_matmul(const NodePtr& root, PreparedGemm& pg) {
        realize(root->parents[0]);
        realize(root->parents[1]);
        pg.n = root;
        pg.out = empty(root->view.shape, DeviceEnum::HIP, DType::Float32);
        pg.empty = pg.out->numel() == 0;
        if (!pg.empty) pg.d = gemm_desc(root, (float*)pg.out->ptr, pg.hold);
    }
    static void matmul_handler(const NodePtr& root) {
        PreparedGemm pg;
        prepare_matmul(root, pg);
        if (!pg.empty && !launch_paired(pg)) ORMI_HIP_CHECK(ormi_hip_gemm_ex(&pg.d, nullptr));
        commit(pg);
    }

    // ------------------------------------------------ GEMM epilogue fusion --
    // An element-wise node whose expression is one of ormi_hip_gemm_ex's
    // epilogues applied to an unrealized 2-D fp32 MATMUL runs as that GEMM,
    // and the product never makes its own round trip through HBM:
    //   D + p*s, D - p*s, p*s - D (and without s)  the SGD update w - grad*lr
    //   f(p), f in relu/tanh/sigmoid/gelu           a forward activation; p is
    //                                               also stored as the
    //                                               MATMUL's buffer (autograd
    //                                               reads it again)
    //   p * f'(D), f' in step/tanh'/sigmoid'/gelu'  an activation's backward
    //   (and p * D)                                 on the dX GEMM
    // D is a realized or non-element-wise node (leaf, view, matmul, reduction),
    // s a one-element fp32 node. The epilogue rounds each operation as the
    // element-wise kernel would, so results are identical either way. A
    // MATMUL left unrealized is computed again if something reads it later.
    // ORMI_GEMM_EPILOGUE=0 (or set_gemm_epilogue(false)) turns the matching off.
    struct EpilogueMatch {
        NodePtr g, d, s;
        int kind = ORMI_GEMM_EPI_NONE, fn = ORMI_GEMM_FN_IDENTITY, form = 0;
    };

    static std::atomic<bool>& epilogue_switch() {
        static std::atomic<bool> on{[] {
            const char* v = std::getenv("ORMI_GEMM_EPILOGUE");
            return !(v && *v && std::atoi(v) == 0);
        }()};
        return on;
    }
    static bool epilogue_enabled() { return epilogue_switch().load(); }
    void set_gemm_epilogue(bool on) { epilogue_switch().store(on); }

    static std::atomic<uint64_t> g_epilogue_gemms{0};
    uint64_t gemm_epilogue_count() { return g_epilogue_gemms.load(); }

    static bool is_open_product(const NodePtr& x, const std::vector<int>& shape) {
        return x->op == OpEnum::MATMUL && !x->is_realized() && x->device.type == DeviceEnum::HIP && x->view.shape == shape &&
               shape.size() == 2 && x->parents[0]->view.shape.size() == 2 && x->parents[1]->view.shape.size() == 2;
    }
    static bool is_scale(const NodePtr& x) {
        return x->dtype == DType::Float32 && shape_numel(x->view.shape) == 1 && (x->is_realized() || !fusible_root(*x));
    }
    // D operand: fp32, broadcasts right-aligned to the 2-D output, already a
    // buffer or produced by a non-element-wise op.
    static bool is_operand(const NodePtr& x, const std::vector<int>& shape) {
        if (x->dtype != DType::Float32 || (!x->is_realized() && fusible_root(*x))) return false;
        const auto& xs = x->view.shape;
        if (xs.size() > shape.size()) return false;
        for (size_t i = 0; i < xs.size(); ++i) {
            const int v = xs[xs.size() - 1 - i];
            if (v != 1 && v != shape[shape.size() - 1 - i]) return false;
        }
        return true;
    }
    static int unary_fn(OpEnum op) {
        switch (op) {
            case OpEnum::RELU: return ORMI_GEMM_FN_RELU;
            case OpEnum::TANH: return ORMI_GEMM_FN_TANH;
            case OpEnum::SIGMOID: return ORMI_GEMM_FN_SIGMOID;
            case OpEnum::GELU: return ORMI_GEMM_FN_GELU;
            default: return -1;
        }
    }
    static int grad_fn(OpEnum op) {
        switch (op) {
            case OpEnum::STEP: return ORMI_GEMM_FN_STEP;
            case OpEnum::TANH_GRAD: return ORMI_GEMM_FN_TANH_GRAD;
            case OpEnum::SIGMOID_GRAD: return ORMI_GEMM_FN_SIGMOID_GRAD;
            case OpEnum::GELU_GRAD: return ORMI_GEMM_FN_GELU_GRAD;
            default: return -1;
        }
    }

    static bool match_epilogue(const NodePtr& n, EpilogueMatch& m) {
        if (!epilogue_enabled() || n->is_realized() || !fusible_root(*n) || n->dtype != DType::Float32) return false;
        const auto& shape = n->view.shape;
        if (shape.size() != 2) return false;
        const NodePtr& x = n->parents[0];
        // p, or p * s / s * p as an unrealized element-wise MUL.
        auto term = [&](const NodePtr& t, NodePtr& g, NodePtr& sc) {
            if (is_open_product(t, shape)) {
                g = t;
                sc = nullptr;
                return true;
            }
            if (t->op != OpEnum::MUL || t->is_realized() || !fusible_interior(*t) || t->dtype != DType::Float32) return false;
            for (int k = 0; k < 2; ++k) {
                const NodePtr &u = t->parents[k], &v = t->parents[1 - k];
                if (is_open_product(u, shape) && is_scale(v)) {
                    g = u;
                    sc = v;
                    return true;
                }
            }
            return false;
        };
        if (n->op == OpEnum::ADD || n->op == OpEnum::SUB) {
            const NodePtr& y = n->parents[1];
            NodePtr g, sc;
            m.kind = ORMI_GEMM_EPI_ADD;
            if (term(y, g, sc) && is_operand(x, shape) && x != g) {
                m.form = n->op == OpEnum::ADD ? 0 : 1;  // D + t, D - t
                m.d = x;
            } else if (term(x, g, sc) && is_operand(y, shape) && y != g) {
                m.form = n->op == OpEnum::ADD ? 0 : 2;  // t + D (= D + t), t - D
                m.d = y;
            } else {
                return false;
            }
            m.g = g;
            m.s = sc;
            return true;
        }
        if (ops::op_arity(n->op) == 1) {
            const int fn = unary_fn(n->op);
            if (fn < 0 || !is_open_product(x, shape)) return false;
            m.kind = ORMI_GEMM_EPI_UNARY;
            m.fn = fn;
            m.g = x;
            return true;
        }
        if (n->op == OpEnum::MUL) {
            for (int k = 0; k < 2; ++k) {
                const NodePtr &u = n->parents[k], &v = n->parents[1 - k];
                if (!is_open_product(u, shape)) continue;
                if (is_operand(v, shape) && v != u) {
                    m.kind = ORMI_GEMM_EPI_MUL_FN_D;
                    m.fn = ORMI_GEMM_FN_IDENTITY;
                    m.g = u;
                    m.d = v;
                    return true;
                }
                const int fn = v->is_realized() || !fusible_interior(*v) ? -1 : grad_fn(v->op);
                if (fn >= 0 && v->dtype == DType::Float32 && is_operand(v->parents[0], shape) && v->parents[0] != u) {
                    m.kind = ORMI_GEMM_EPI_MUL_FN_D;
                    m.fn = fn;
                    m.g = u;
                    m.d = v->parents[0];
                    return true;
                }
            }
        }
        return false;
    }

    // Prepare n as its matched GEMM; false (nothing prepared) when a realized
    // operand turns out not to be fp32.
    static bool prepare_epilogue(const NodePtr& n, const EpilogueMatch& m, PreparedGemm& pg) {
        if (m.d) realize(m.d);
        if (m.s) realize(m.s);
        if ((m.d && m.d->data->dtype != DType::Float32) || (m.s && m.s->data->dtype != DType::Float32)) return false;
        ormi_gemm_epilogue& e = pg.e;
        e.kind = m.kind;
        e.fn = m.fn;
        e.form = m.form;
        if (m.s) e.s = (const float*)m.s->data->ptr;
        if (m.d) {
            e.d = (const float*)m.d->data->ptr;
            const auto& ds = m.d->view.shape;
            const auto& dst = m.d->view.strides;
            const bool scalar = ds.empty() || m.d->data->numel() == 1;
            int64_t st[2] = {0, 0};
            for (size_t i = 0; i < ds.size() && !scalar; ++i) {
                const size_t p = 2 - ds.size() + i;
                if (ds[i] != 1) st[p] = dst[i];
            }
            e.d_stride_m = st[0];
            e.d_stride_n = st[1];
        }
        pg.n = n;
        pg.g = m.g;
        pg.hold = {m.d, m.s};
        pg.out = empty(n->view.shape, DeviceEnum::HIP, DType::Float32);
        if (m.kind == ORMI_GEMM_EPI_UNARY) {
            pg.aux = empty(m.g->view.shape, DeviceEnum::HIP, DType::Float32);
            e.aux = (float*)pg.aux->ptr;
        }
        pg.empty = pg.out->numel() == 0;
        if (!pg.empty) pg.d = gemm_desc(m.g, (float*)pg.out->ptr, pg.hold);
        return true;
    }

    static void commit(PreparedGemm& pg) {
        pg.n->data = pg.out;
        pg.n->view.strides = calc_contiguous_strides(pg.n->view.shape);
        if (pg.aux) {
            pg.g->data = pg.aux;
            pg.g->view.strides = calc_contiguous_strides(pg.g->view.shape);
        }
        if (pg.g) g_epilogue_gemms.fetch_add(1);
    }

    // Run n as its matched GEMM; false (nothing launched) when a realized
    // operand turns out not to be fp32.
    static bool run_gemm_epilogue(const NodePtr& n, const EpilogueMatch& m) {
        PreparedGemm pg;
        if (!prepare_epilogue(n, m, pg)) return false;
        if (!pg.empty && !launch_paired(pg)) ORMI_HIP_CHECK(ormi_hip_gemm_ex(&pg.d, &pg.e));
        commit(pg);
        return true;
    }

    // Forward activations of GEMM products, indexed once per top-level
    // realize. Autograd can reach a product p first through f'(p), as the D of
    // a backward epilogue, when a weight update is realized before the loss;
    // p would then run as a plain GEMM and f(p) as a map over it. A product the
    // scheduler must compute runs instead as the UNARY epilogue of an
    // activation f(p) the same graph holds, which stores p and f(p) from one
    // GEMM (identical values either way).
    struct RealizeScope {
        const NodePtr* roots = nullptr;  // the outermost call's roots, alive for the scope
        size_t nroots = 0;
        bool indexed = false;
        std::unordered_map<Node*, NodePtr> act;  // product -> f(product)
        bool gemms_indexed = false;
        std::vector<NodePtr> gemms;  // products the scope will realize (pairing candidates)
    };
    static thread_local RealizeScope* t_scope = nullptr;
    // The outermost realize owns the scope; nested realizes share it.
    struct ScopeGuard {
        RealizeScope scope;
        bool owner;
        // The roots belong to the outermost caller, which outlives the scope.
        ScopeGuard(const NodePtr* roots, size_t n) : owner(t_scope == nullptr) {
            if (!owner) return;
            scope.roots = roots;
            scope.nroots = n;
            t_scope = &scope;
        }
        ~ScopeGuard() {
            if (owner) t_scope = nullptr;
        }
        ScopeGuard(const ScopeGuard&) = delete;
        ScopeGuard& operator=(const ScopeGuard&) = delete;
    };

    static NodePtr activation_consumer(const NodePtr& p) {
        if (!t_scope || !epilogue_enabled()) return nullptr;
        RealizeScope& sc = *t_scope;
        if (!sc.indexed) {
            // Walk the unrealized part of the graph below the roots once.
            sc.indexed = true;
            std::vector<NodePtr> stack;
            std::unordered_set<Node*> seen;
            for (size_t i = 0; i < sc.nroots; ++i) {
                const NodePtr& r = sc.roots[i];
                if (r && !r->is_realized() && seen.insert(r.get()).second) stack.push_back(r);
            }
            while (!stack.empty()) {
                const NodePtr n = stack.back();
                stack.pop_back();
                if (ops::op_arity(n->op) == 1 && unary_fn(n->op) >= 0 && fusible_root(*n) && n->dtype == DType::Float32 &&
                    is_open_product(n->parents[0], n->view.shape))
                    sc.act.emplace(n->parents[0].get(), n);
                for (const auto& q : n->parents)
                    if (!q->is_realized() && seen.insert(q.get()).second) stack.push_back(q);
            }
        }
        const auto it = sc.act.find(p.get());
        return it == sc.act.end() || it->second->is_realized() ? nullptr : it->second;
    }

    // ------------------------------------------------------ GEMM pairing --
    // The backward of a MATMUL builds two products on one dZ, dX = dZ Y^T and
    // dY = X^T dZ (reference csrc/core/ops/blas/matmul.cpp:84-124); in a
    // training step dX (often with an activation's derivative, a MUL_FN_D
    // epilogue) feeds the layer below while dY feeds the weight update (an ADD
    // epilogue). The two are independent, so when the scheduler is about to
    // launch one, another product of the same realize scope whose inputs are
    // all realized runs with it through ormi_hip_gemm_pair: one persistent
    // launch when the library can group them, else two calls in order. The
    // results are the same bits either way; only when the partner's buffer is
    // filled changes. ORMI_GEMM_PAIR=0 (read by the library on each call) keeps
    // the launches separate.
    static std::atomic<uint64_t> g_gemm_pairs{0};
    uint64_t gemm_pair_count() { return g_gemm_pairs.load(); }

    // Whether a product of this 2-D shape, depth and epilogue kind is one the
    // library can group: fp32, whole 128x128 tiles, K in whole 32-deep tiles,
    // at least one tile per compute unit, no activation epilogue. The library
    // checks the rest (layouts, strides, independence).
    static bool pair_shape(long long M, long long N, long long K, int kind) {
        return M > 0 && N > 0 && K > 0 && M % 128 == 0 && N % 128 == 0 && K % 32 == 0 &&
               (M / 128) * (N / 128) >= device_compute_units() && kind != ORMI_GEMM_EPI_UNARY;
    }
    static bool pair_candidate_shape(const NodePtr& g, int kind) {
        const auto& a = g->parents[0];
        const auto& b = g->parents[1];
        if (g->view.shape.size() != 2 || a->dtype != DType::Float32 || b->dtype != DType::Float32) return false;
        return pair_shape(g->view.shape[0], g->view.shape[1], a->view.shape.back(), kind);
    }

    // x holds a buffer, or is a chain of views over one that does.
    static bool realized_through_views(NodePtr x) {
        while (!x->is_realized() && is_view_op(x->op)) x = x->parents[0];
        return x->is_realized();
    }

    static const std::vector<NodePtr>& scope_gemms(RealizeScope& sc) {
        if (sc.gemms_indexed) return sc.gemms;
        sc.gemms_indexed = true;
        // The roots and every operand of a MATMUL below them: nodes the scope
        // realizes whatever the order.
        std::vector<NodePtr> stack, found;
        std::unordered_set<Node*> seen, taken;
        auto take = [&](const NodePtr& c) {
            if (!c->is_realized() && taken.insert(c.get()).second) found.push_back(c);
        };
        for (size_t i = 0; i < sc.nroots; ++i) {
            const NodePtr& r = sc.roots[i];
            if (!r || r->is_realized()) continue;
            take(r);
            if (seen.insert(r.get()).second) stack.push_back(r);
        }
        while (!stack.empty()) {
            const NodePtr n = stack.back();
            stack.pop_back();
            if (n->op == OpEnum::MATMUL)
                for (const auto& q : n->parents) take(q);
            for (const auto& q : n->parents)
                if (!q->is_realized() && seen.insert(q.get()).second) stack.push_back(q);
        }
        for (const auto& c : found) {
            EpilogueMatch m;
            const bool gemm = c->op == OpEnum::MATMUL || (c->device.type == DeviceEnum::HIP && match_epilogue(c, m));
            if (gemm && c->device.type == DeviceEnum::HIP) sc.gemms.push_back(c);
        }
        return sc.gemms;
    }

    static std::vector<NodePtr> dependencies(const NodePtr& n);

    // Launch self together with a ready partner from the scope; false (nothing
    // launched) when there is none.
    static bool launch_paired(PreparedGemm& self) {
        if (!t_scope || self.empty) return false;
        const ormi_gemm_desc& d = self.d;
        if (d.dtype != ORMI_DTYPE_F32 || d.batch_ndim != 0 || !pair_shape(d.M, d.N, d.K, self.e.kind)) return false;
        const Node* self_product = self.g ? self.g.get() : self.n.get();
        for (const NodePtr& c : scope_gemms(*t_scope)) {
            if (c->is_realized() || c == self.n) continue;
            EpilogueMatch m;
            const bool epi = c->op != OpEnum::MATMUL;
            if (epi && !match_epilogue(c, m)) continue;
            const NodePtr& g = epi ? m.g : c;
            if (g.get() == self_product || g->is_realized()) continue;
            // A product whose activation the scope holds runs as that
            // activation's epilogue (it stores both), not as a plain GEMM.
            if (!epi && activation_consumer(c)) continue;
            if (!pair_candidate_shape(g, epi ? m.kind : ORMI_GEMM_EPI_NONE)) continue;
            bool ready = true;
            for (const auto& dep : dependencies(c)) ready = ready && realized_through_views(dep);
            if (!ready) continue;
            PreparedGemm other;
            if (epi) {
                if (!prepare_epilogue(c, m, other)) continue;
            } else {
                prepare_matmul(c, other);
            }
            if (other.empty) {
                commit(other);
                continue;
            }
            int grouped = 0;
            ORMI_HIP_CHECK(ormi_hip_gemm_pair(&self.d, &self.e, &other.d, epi ? &other.e : nullptr, &grouped));
            if (grouped) g_gemm_pairs.fetch_add(1);
            commit(other);
            return true;
        }
        return false;
    }

    // An element-wise region: a matched GEMM epilogue, a reduction's store
    // epilogue, else one fused kernel.
    static void run_map(const NodePtr& root) {
        {
            EpilogueMatch m;
            if (match_epilogue(root, m) && run_gemm_epilogue(root, m)) return;
        }
        if (const NodePtr r = epilogue_reduction(root)) {
            reduce_handler(r, r->op == OpEnum::SUM ? ReduceOp::Sum : ReduceOp::Max, root);
            return;
        }
        for (const auto& f : region_frontier(root)) realize(f);
        const Expr e = build_expr(root, root->view.shape);
        auto out = empty(root->view.shape, DeviceEnum::HIP, root->dtype);
        root->data = out;
        root->view.strides = calc_contiguous_strides(root->view.shape);
        if (out->numel() == 0) return;
        launch(plan_map(e, root->view.shape, out->ptr, root->dtype, device_compute_units(), true));
    }

    // Nodes that must hold buffers before `n` can run as one step: a view's
    // parent, an element-wise region's frontier, the frontier (or the input)
    // of a reduction, a matmul's operands.
    static std::vector<NodePtr> dependencies(const NodePtr& n) {
        if (is_view_op(n->op)) return {n->parents[0]};
        if (fusible_root(*n)) {
            EpilogueMatch m;
            if (match_epilogue(n, m)) {
                std::vector<NodePtr> deps{m.g->parents[0], m.g->parents[1]};
                if (m.d) deps.push_back(m.d);
                if (m.s) deps.push_back(m.s);
                return deps;
            }
            if (const NodePtr r = epilogue_reduction(n)) return dependencies(r);
            return region_frontier(n);
        }
        if (ops::is_reduction(n->op)) {
            const NodePtr& x = n->parents[0];
            if (fuse_as_prologue(x)) return region_frontier(x);
            return {x};
        }
        return n->parents;
    }

    // One node whose dependencies are realized.
    static void realize_one(const NodePtr& n) {
        if (n->device.type != DeviceEnum::HIP) throw std::runtime_error("HIP scheduler: node belongs to another device.");
        if (is_view_op(n->op)) {
            n->data = n->parents[0]->data;
            return;
        }
        if (fusible_root(*n)) {
            run_map(n);
            return;
        }
        if (n->op == OpEnum::MATMUL) {
            // Its operands are realized, and so are the activation's (the same).
            if (const NodePtr a = activation_consumer(n)) {
                EpilogueMatch m;
                if (match_epilogue(a, m) && m.g == n && run_gemm_epilogue(a, m) && n->is_realized()) return;
            }
        }
        if (try_execute_graph_break(n)) return;
        if (n->op == OpEnum::LEAF || n->op == OpEnum::CONST) throw std::runtime_error("HIP scheduler: leaf without a buffer.");
        throw std::runtime_error(std::string("HIP scheduler: no lowering for op ") + ops::op_name(n->op));
    }

    // Post-order over dependencies with an explicit stack, so chains of any
    // length (an unrolled recurrence of matmuls and reductions) need no deep
    // recursion. A region's frontier only shrinks as nodes get buffers, so the
    // dependencies pushed for a node still cover it when it runs.
    void realize(const NodePtr& root) {
        if (!root || root->is_realized()) return;
        ScopeGuard guard(&root, 1);
        SmallVec<NodePtr, 16> stack;
        stack.push_back(root);
        SmallSet<Node> expanded;
        while (!stack.empty()) {
            const NodePtr n = stack.back();
            if (n->is_realized()) {
                stack.pop_back();
                continue;
            }
            if (expanded.insert(n.get())) {
                bool pushed = false;
                for (const auto& d : dependencies(n)) {
                    if (d->is_realized()) continue;
                    stack.push_back(d);
                    pushed = true;
                }
                if (pushed) continue;
            }
            stack.pop_back();
            realize_one(n);
        }
    }

    void realize_group(const std::vector<NodePtr>& roots) {
        ScopeGuard guard(roots.data(), roots.size());
        // Element-wise roots with float results that can share one kernel,
        // grouped by shape in first-seen order; everything else realizes alone.
        std::vector<std::pair<std::vector<int>, std::vector<NodePtr>>> groups;
        std::vector<NodePtr> rest;
        std::unordered_set<Node*> seen;
        for (const auto& r : roots) {
            if (!r || r->is_realized() || !seen.insert(r.get()).second) continue;
            if (r->device.type != DeviceEnum::HIP) throw std::runtime_error("HIP scheduler: node belongs to another device.");
            EpilogueMatch m;
            if (!fusible_interior(*r) || match_epilogue(r, m) || epilogue_reduction(r)) {
                rest.push_back(r);
                continue;
            }
            auto it = std::find_if(groups.begin(), groups.end(), [&](const auto& g) { return g.first == r->view.shape; });
            if (it == groups.end()) groups.push_back({r->view.shape, {r}});
            else it->second.push_back(r);
        }
        for (auto& [shape, members] : groups) {
            for (const auto& m : members)
                for (const auto& f : region_frontier(m)) realize(f);
            std::vector<NodePtr> live;
            for (const auto& m : members)
                if (!m->is_realized()) live.push_back(m);
            if (live.empty()) continue;
            if (live.size() == 1) {
                run_map(live[0]);
                continue;
            }
            // The tape is built while every member is still unrealized, so a
            // member inside another's region stays an instruction, not a leaf.
            const Expr e = build_expr_multi(live, shape);
            std::vector<std::shared_ptr<Buffer>> bufs;
            std::vector<void*> outs;
            std::vector<DType> dts;
            for (const auto& m : live) {
                bufs.push_back(empty(m->view.shape, DeviceEnum::HIP, m->dtype));
                outs.push_back(bufs.back()->ptr);
                dts.push_back(m->dtype);
            }
            if (shape_numel(shape) > 0) launch(plan_map_multi(e, shape, outs, dts, device_compute_units(), true));
            for (size_t i = 0; i < live.size(); ++i) {
                live[i]->data = bufs[i];
                live[i]->view.strides = calc_contiguous_strides(live[i]->view.shape);
            }
        }
        for (const auto& r : rest) realize(r);
    }

    static RegisterGraphBreaker reg_sum(DeviceEnum::HIP, OpEnum::SUM, [](std::shared_ptr<Node> n) { reduce_handler(n, ReduceOp::Sum); });
    static RegisterGraphBreaker reg_max(DeviceEnum::HIP, OpEnum::MAX, [](std::shared_ptr<Node> n) { reduce_handler(n, ReduceOp::Max); });
    static RegisterGraphBreaker reg_argmax(DeviceEnum::HIP, OpEnum::ARGMAX, [](std::shared_ptr<Node> n) { reduce_handler(n, ReduceOp::Argmax); });
    static RegisterGraphBreaker reg_matmul(DeviceEnum::HIP, OpEnum::MATMUL, matmul_handler);
    static RegisterScheduler reg_sched(DeviceEnum::HIP, [](std::shared_ptr<Node> n) { realize(n); });
    static RegisterGroupScheduler reg_group(DeviceEnum::HIP, [](const std::vector<std::shared_ptr<Node>>& ns) { realize_group(ns); });
    // Element-wise JIT entry for a node whose parents are realized: the
    // reference's execute_jit slot (csrc/backend/runtime.cpp:29-38).
    static RegisterJit reg_jit(DeviceEnum::HIP, [](std::shared_ptr<Node> n) { run_map(n); });
}
