// hipRTC code generator for gfx950: fused element-wise maps, and row / column
// reductions with a fused element-wise prologue.
//
// Replaces the reference's NVRTC source builder (csrc/backend/cuda/compiler.cu:53-112)
// and its atomic sum kernel (csrc/backend/cuda/kernels/reduce/sum.cu:29-66). Unlike
// those, sizes and strides are kernel arguments (never literals), so a kernel is
// reused for every tensor with the same structure; the source only encodes the
// tape, operand dtypes, which strides are 0 or 1, the vector width and the
// index width. A structural signature of exactly those choices keys a cache of
// generated kernels, so a repeat launch builds its argument list and nothing else.
//
// Index space. The kernel's logical shape is canonicalized first: size-1 dims are
// dropped and neighbouring dims merged wherever every operand (and the output)
// is linear across them. A reduction splits its dims into three groups, kept
// dims before the last reduced one (O), reduced dims (R) and kept dims after it
// (I), so out[o][i] = reduce_r f(o, r, i) with a contiguous output.
//   * map:     each thread handles UNROLL groups of VEC (4) consecutive
//              elements: 128-bit loads and stores, grid-stride over tiles
//              sized for the chip's compute units.
//   * row:     I empty. One wave64 per (row, part): lanes stride the row with
//              128-bit loads, then a DPP/cross-lane wave reduction.
//   * column:  I non-empty. 64 lanes along I (128-bit loads), W waves split R;
//              the W partials are combined through LDS in wave order.
// When O (or O x I) is too small to fill 256 CUs, R is split into parts whose
// partial results go to a workspace, and a second kernel combines them in part
// order (two-pass; deterministic, no atomics).
#include <algorithm>
#include <atomic>
#include <charconv>
#include <memory>
#include <cstdlib>
#include <mutex>
#include <sstream>
#include <string_view>
#include <unordered_map>

#include "backend/hip/kernel_gen.h"

namespace ormi::hip {
    using ops::OpEnum;

    const LoweringFunc* builtin_lowering(OpEnum op) {
        using A = const std::vector<std::string>&;
        static const std::unordered_map<OpEnum, LoweringFunc> table = {
            {OpEnum::ADD, [](A v) { return "(" + v[0] + " + " + v[1] + ")"; }},
            {OpEnum::SUB, [](A v) { return "(" + v[0] + " - " + v[1] + ")"; }},
            {OpEnum::MUL, [](A v) { return "(" + v[0] + " * " + v[1] + ")"; }},
            {OpEnum::DIV, [](A v) { return "(" + v[0] + " / " + v[1] + ")"; }},
            {OpEnum::POW, [](A v) { return "powf(" + v[0] + ", " + v[1] + ")"; }},
            {OpEnum::EQ, [](A v) { return "ormi_eq(" + v[0] + ", " + v[1] + ")"; }},
            {OpEnum::NEG, [](A v) { return "(-" + v[0] + ")"; }},
            {OpEnum::EXP, [](A v) { return "ormi_exp(" + v[0] + ")"; }},
            {OpEnum::LOG, [](A v) { return "logf(" + v[0] + ")"; }},
            {OpEnum::SIN, [](A v) { return "sinf(" + v[0] + ")"; }},
            {OpEnum::COS, [](A v) { return "cosf(" + v[0] + ")"; }},
            {OpEnum::RELU, [](A v) { return "ormi_relu(" + v[0] + ")"; }},
            {OpEnum::STEP, [](A v) { return "ormi_step(" + v[0] + ")"; }},
            {OpEnum::TANH, [](A v) { return "ormi_tanh(" + v[0] + ")"; }},
            {OpEnum::TANH_GRAD, [](A v) { return "ormi_tanh_grad(" + v[0] + ")"; }},
            {OpEnum::SIGMOID, [](A v) { return "ormi_sigmoid(" + v[0] + ")"; }},
            {OpEnum::SIGMOID_GRAD, [](A v) { return "ormi_sigmoid_grad(" + v[0] + ")"; }},
            {OpEnum::GELU, [](A v) { return "ormi_gelu(" + v[0] + ")"; }},
            {OpEnum::GELU_GRAD, [](A v) { return "ormi_gelu_grad(" + v[0] + ")"; }},
        };
        auto it = table.find(op);
        return it == table.end() ? nullptr : &it->second;
    }

    static const char* kDeviceHeader =
#include "ormi_device_text.inc"
        ;

    const std::vector<std::string>& rtc_options() {
        // Packed-FP32 instructions stay disabled in generated code as in every
        // hipcc-built translation unit.
        static const std::vector<std::string> opts = {"-O3", "-std=c++17", "-ffp-contract=off",
                                                      "-fhip-fp32-correctly-rounded-divide-sqrt",
                                                      "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
        return opts;
    }

    static int env_int(const char* name, int dflt) {
        const char* v = std::getenv(name);
        return v && *v ? std::atoi(v) : dflt;
    }

    const Tuning& tuning() {
        static const Tuning t = [] {
            Tuning x;
            x.map_unroll = std::clamp(env_int("ORMI_MAP_UNROLL", x.map_unroll), 1, 8);
            x.map_blocks_per_cu = std::clamp(env_int("ORMI_MAP_BLOCKS_PER_CU", x.map_blocks_per_cu), 1, 1024);
            x.row_unroll = std::clamp(env_int("ORMI_ROW_UNROLL", x.row_unroll), 1, 8);
            x.row_waves = env_int("ORMI_ROW_WAVES", x.row_waves);
            if (x.row_waves != 1 && x.row_waves != 2 && x.row_waves != 4) x.row_waves = 4;
            x.row_waves_min_groups = std::max(1, env_int("ORMI_ROW_WAVES_MIN_GROUPS", x.row_waves_min_groups));
            x.col_waves = std::clamp(env_int("ORMI_COL_WAVES", x.col_waves), 1, 16);
            x.col_cwaves = std::clamp(env_int("ORMI_COL_CWAVES", x.col_cwaves), 1, 16);
            x.col_unroll = std::clamp(env_int("ORMI_COL_UNROLL", x.col_unroll), 1, 8);
            x.col_fin_split = env_int("ORMI_COL_FIN_SPLIT", x.col_fin_split);
            if (x.col_fin_split != 1 && x.col_fin_split != 2 && x.col_fin_split != 4 && x.col_fin_split != 8) x.col_fin_split = 1;
            x.map_wg_per_cu = std::clamp(env_int("ORMI_MAP_WG_PER_CU", x.map_wg_per_cu), 0, 32);
            x.map_row_tile_wg_per_cu = std::clamp(env_int("ORMI_MAP_ROW_TILE_WG_PER_CU", x.map_row_tile_wg_per_cu), 0, 32);
            x.row_wg_per_cu = std::clamp(env_int("ORMI_ROW_WG_PER_CU", x.row_wg_per_cu), 0, 32);
            x.row_max_wg_per_cu = std::clamp(env_int("ORMI_ROW_MAX_WG_PER_CU", x.row_max_wg_per_cu), 0, 32);
            x.map_nt_loads = env_int("ORMI_MAP_NT_LOADS", x.map_nt_loads) != 0;
            x.reduce_nt_loads = env_int("ORMI_REDUCE_NT_LOADS", x.reduce_nt_loads) != 0;
            x.nt_min_bytes = std::max(0, env_int("ORMI_NT_MIN_MIB", (int)(x.nt_min_bytes >> 20))) * (1LL << 20);
            x.map_nt_stores = env_int("ORMI_MAP_NT_STORES", x.map_nt_stores) != 0;
            x.map_off32 = env_int("ORMI_MAP_OFF32", x.map_off32) != 0;
            x.map_rows = env_int("ORMI_MAP_ROWS", x.map_rows) != 0;
            x.map_row_tiles = env_int("ORMI_MAP_ROW_TILES", x.map_row_tiles) != 0;
            return x;
        }();
        return t;
    }

    // Dynamic LDS that lets at most n work-groups of a kernel share one CU
    // (gfx950: 160 KB of LDS per CU, allocated in 512-byte units), leaving
    // 1 KB per work-group for the kernel's own LDS; 0 when n is 0 or the grid
    // would not fill n per CU anyway. Fewer concurrent streams use HBM better
    // where a kernel writes about as much as it reads, or where its
    // work-groups read long streams, down to the point where too few waves
    // are left to cover the arithmetic. Short-lived read-only work-groups
    // need every slot instead (a one-shot 8 KB read per work-group: 7.13 TB/s
    // uncapped, 6.37 at 5 per CU, 4.25 at 3). Measured on C2's shapes: the
    // copy y = -x took 43.7-43.8 us at the 8 per CU its registers allow and
    // 42.0-42.3 at 5; C2's chain 44.4 at 8, 44.1 at 5, 45.4-45.6 at 4. C3's
    // row sum with four waves per 32 KB row took 79.7-80.2 us at 8 and
    // 76.1-76.4 at 3; its row max 80.3-80.4 at 8, 75.9-76.1 at 4 and
    // 82.1-82.4 at 3 (each element extends a dependent (value, index) chain).
    static uint32_t occupancy_lds(int n, long long grid, int cu) {
        if (n <= 0 || grid <= (long long)n * std::max(cu, 1)) return 0;
        constexpr int kCuLds = 160 * 1024;
        return (uint32_t)((kCuLds / n - 1024) / 512 * 512);
    }

    FastDiv make_fastdiv(uint32_t d) {
        if (d == 0) throw std::runtime_error("fastdiv by zero");
        if (d > (1u << 31)) throw std::runtime_error("fastdiv divisor above 2^31");
        uint32_t s = 0;
        while ((1ull << s) < d) ++s;
        const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
        return FastDiv{d, (uint32_t)m, s};
    }

    namespace {
        const char* storage_type(DType t) {
            switch (t) {
                case DType::Float32: return "float";
                case DType::BFloat16: case DType::Float16: return "unsigned short";
                case DType::Int64: return "long long";
                case DType::Int32: return "int";
                case DType::Bool: return "unsigned char";
            }
            return "float";
        }

        bool vector_dtype(DType t) { return t == DType::Float32 || t == DType::BFloat16 || t == DType::Float16; }

        std::string to_f32(DType t, const std::string& v) {
            switch (t) {
                case DType::Float32: return v;
                case DType::BFloat16: return "ormi_bf16_to_f32(" + v + ")";
                case DType::Float16: return "ormi_f16_to_f32(" + v + ")";
                case DType::Bool: return "((" + v + ") ? 1.0f : 0.0f)";
                default: return "((float)(" + v + "))";
            }
        }

        std::string from_f32(DType t, const std::string& v) {
            switch (t) {
                case DType::Float32: return v;
                case DType::BFloat16: return "ormi_f32_to_bf16(" + v + ")";
                case DType::Float16: return "ormi_f32_to_f16(" + v + ")";
                case DType::Int64: return "ormi_f32_to_i64(" + v + ")";
                case DType::Int32: return "ormi_f32_to_i32(" + v + ")";
                case DType::Bool: return "((unsigned char)((" + v + ") != 0.0f))";
            }
            return v;
        }

        // Canonical index space: dims in kernel order with their group tag.
        enum Group { G_O = 0, G_R = 1, G_I = 2, G_M = 3 };
        struct Dim {
            long long size;
            Group group;
        };
        struct Canon {
            std::vector<Dim> dims;
            std::vector<std::vector<long long>> st;  // [leaf][dim]
        };

        // Drop size-1 dims, then merge dim d into d+1 when both are in the same
        // group and every operand is linear across them. Output contiguity is
        // preserved because groups keep the output's dim order.
        void canonicalize(Canon& c, const std::vector<bool>& scalar) {
            Canon out;
            out.st.resize(c.st.size());
            for (size_t d = 0; d < c.dims.size(); ++d) {
                if (c.dims[d].size == 1) continue;
                out.dims.push_back(c.dims[d]);
                for (size_t L = 0; L < c.st.size(); ++L) out.st[L].push_back(c.st[L][d]);
            }
            bool merged = true;
            while (merged) {
                merged = false;
                for (size_t d = 0; d + 1 < out.dims.size(); ++d) {
                    if (out.dims[d].group != out.dims[d + 1].group) continue;
                    bool ok = true;
                    for (size_t L = 0; L < out.st.size() && ok; ++L)
                        if (!scalar[L]) ok = out.st[L][d] == out.st[L][d + 1] * out.dims[d + 1].size;
                    if (!ok) continue;
                    out.dims[d].size *= out.dims[d + 1].size;
                    out.dims.erase(out.dims.begin() + d + 1);
                    for (auto& s : out.st) {
                        s[d] = s[d + 1];
                        s.erase(s.begin() + d + 1);
                    }
                    merged = true;
                    break;
                }
            }
            c = std::move(out);
        }

        // A kernel parameter. Its declaration text is rendered only when a
        // source is generated (a cache miss); signatures use the fields.
        struct ArgDecl {
            bool is_const;
            const char* type;  // storage type literal: "float", "long long", ...
            bool is_ptr;
            const char* name;  // name literal, followed by i and _j when >= 0
            int i, j;
        };
        std::string render(const ArgDecl& d) {
            std::string r = d.is_const ? "const " : "";
            r += d.type;
            r += d.is_ptr ? "* __restrict__ " : " ";
            r += d.name;
            if (d.i >= 0) r += std::to_string(d.i);
            if (d.j >= 0) r += "_" + std::to_string(d.j);
            return r;
        }

        struct ArgList {
            std::vector<ArgDecl> decls;
            std::vector<uint64_t> vals;
            void ptr(bool is_const, const char* type, const char* name, const void* p, int i = -1) {
                decls.push_back({is_const, type, true, name, i, -1});
                vals.push_back((uint64_t)(uintptr_t)p);
            }
            void i64(const char* name, long long v, int i = -1, int j = -1) {
                decls.push_back({true, "long long", false, name, i, j});
                vals.push_back((uint64_t)v);
            }
        };

        // ptr_slots source of a store epilogue's leaf i (see resolve).
        constexpr int kEpilogueLeaf = 1 << 20;

        // Appends without stream machinery (the signature is built per launch).
        void append_int(std::string& s, long long v) {
            char buf[24];
            auto r = std::to_chars(buf, buf + sizeof(buf), v);
            s.append(buf, r.ptr);
        }

        std::string hex_hash(const std::string& s) {
            uint64_t h = 1469598103934665603ull;
            for (unsigned char ch : s) {
                h ^= ch;
                h *= 1099511628211ull;
            }
            std::ostringstream o;
            o << std::hex << h;
            return o.str();
        }

        // Shared pieces of every generated kernel.
        struct Gen {
            const Expr& e;
            Canon c;
            std::vector<bool> scalar;
            bool idx32 = true;
            // off32 (map kernels that ask for it, idx32 only): every operand and
            // output byte offset fits in 32 bits. Indices are unsigned and each
            // access is base pointer + 32-bit byte offset, which the compiler
            // emits as a load or store with a uniform (SGPR) base and a 32-bit
            // VGPR offset, with no 64-bit address arithmetic per element.
            bool want_off32 = false;
            bool off32 = false;
            int vec = 1;
            int vec_dim = -1;  // dim whose coordinate advances by VEC
            int rows = 0;      // map tile alignment to the last dim (plan_map_multi)
            // Non-temporal hint on the loads of streamed leaves: those with no
            // zero stride in the canonical (size-1-free) dims, whose elements
            // the kernel reads once. A broadcast leaf (a bias row re-read by
            // every row) keeps plain loads, so its lines stay in the L2.
            bool nt_loads = false;
            bool streamed(size_t L) const {
                for (long long s : c.st[L])
                    if (s == 0) return false;
                return true;
            }
            // Bytes the streamed leaves bring in over `numel` kernel elements.
            long long streamed_bytes(long long numel) const {
                long long b = 0;
                for (size_t L = 0; L < e.leaves.size(); ++L)
                    if (!scalar[L] && streamed(L)) b += numel * (long long)dtype_size(e.leaves[L].dtype);
                return b;
            }
            // The hint pays on streams larger than the caches (measured on a
            // 128 MiB copy: 45.4 -> 43.5 us). On small operands, which the
            // Infinity Cache may still hold from their producer, it costs.
            void choose_nt_loads(bool enabled, long long numel) {
                nt_loads = enabled && streamed_bytes(numel) >= tuning().nt_min_bytes;
            }
            // Output dtypes of a map: bf16 and fp16 share a storage type, so the
            // argument list alone does not tell their stores apart.
            std::vector<DType> out_dtypes;
            ArgList args;
            std::unique_ptr<std::ostringstream> body_;  // created when a source is generated

            std::ostringstream& body() {
                if (!body_) body_ = std::make_unique<std::ostringstream>();
                return *body_;
            }

            explicit Gen(const Expr& ex) : e(ex) {
                for (const auto& L : e.leaves) scalar.push_back(L.scalar);
            }

            std::string idx() const { return off32 ? "unsigned" : idx32 ? "int" : "long long"; }

            // Pointer expression for element `off` of pointer `base` of type T
            // (sizeof `bytes`), cast to `ptr_type`.
            std::string elem_ptr(const std::string& ptr_type, const std::string& base, const std::string& off, int bytes,
                                 bool is_const) const {
                if (!off32) return "(" + ptr_type + ")(" + base + " + (" + off + "))";
                return "(" + ptr_type + ")((" + (is_const ? "const char*" : "char*") + ")" + base + " + (unsigned)(" + off +
                       ") * " + std::to_string(bytes) + "u)";
            }

            // Leaf L has a unit stride on the vector dim and can be read 4-wide.
            bool leaf_vec_ok(size_t L, int d) const {
                if (scalar[L]) return true;
                const long long s = c.st[L][d];
                if (s == 0) return true;
                if (s != 1 || !vector_dtype(e.leaves[L].dtype)) return false;
                for (size_t k = 0; k < c.dims.size(); ++k)
                    if ((int)k != d && c.st[L][k] % 4 != 0) return false;
                return ((uintptr_t)e.leaves[L].ptr % (4 * dtype_size(e.leaves[L].dtype))) == 0;
            }

            void choose_vec(int d) {
                vec = 1;
                vec_dim = d;
                if (d < 0 || c.dims[d].size % 4 != 0) return;
                for (size_t L = 0; L < e.leaves.size(); ++L)
                    if (!leaf_vec_ok(L, d)) return;
                vec = 4;
            }

            // 32-bit index arithmetic when every index the kernel forms (element
            // counts, operand offsets, the cursor bound extra_extent) fits.
            // out_bytes: largest output element size (for off32).
            void choose_idx(long long extra_extent, int out_bytes = 4) {
                const long long lim = (1ll << 31) - 1;
                const long long blim = (1ll << 32) - 1;
                long long numel = 1;
                for (auto& d : c.dims) numel *= d.size;
                idx32 = numel < lim && extra_extent < lim;
                off32 = want_off32 && idx32 && (numel + 4) * out_bytes < blim;
                for (size_t L = 0; L < e.leaves.size() && idx32; ++L) {
                    if (scalar[L]) continue;
                    long long span = 0;
                    bool nonneg = true;
                    for (size_t d = 0; d < c.dims.size(); ++d) {
                        span += (c.dims[d].size - 1) * std::llabs(c.st[L][d]);
                        nonneg = nonneg && c.st[L][d] >= 0;
                    }
                    if (span >= lim) idx32 = false;
                    if (!nonneg || (span + 4) * dtype_size(e.leaves[L].dtype) >= blim) off32 = false;
                }
                off32 = off32 && idx32;
            }

            void declare_leaves() {
                for (size_t L = 0; L < e.leaves.size(); ++L)
                    args.ptr(true, storage_type(e.leaves[L].dtype), "L", e.leaves[L].ptr, (int)L);
            }

            // Size (in VEC groups for the vector dim) and fastdiv magic of each dim.
            void declare_dims() {
                for (size_t d = 0; d < c.dims.size(); ++d) {
                    const long long n = (int)d == vec_dim ? c.dims[d].size / vec : c.dims[d].size;
                    args.i64("D", n, (int)d);
                    if (idx32) {
                        const FastDiv f = make_fastdiv((uint32_t)n);
                        args.i64("M", (long long)((uint64_t)f.m | ((uint64_t)f.s << 32)), (int)d);
                    }
                }
            }

            // Runtime strides for the dims where they are neither 0 nor 1.
            void declare_strides() {
                for (size_t L = 0; L < e.leaves.size(); ++L) {
                    if (scalar[L]) continue;
                    for (size_t d = 0; d < c.dims.size(); ++d) {
                        const long long s = c.st[L][d];
                        if (s != 0 && s != 1) args.i64("S", s, (int)L, (int)d);
                    }
                }
            }

            std::string stride_term(size_t L, size_t d) const {
                const long long s = c.st[L][d];
                const std::string cd = "c" + std::to_string(d);
                if (s == 0) return "";
                if (s == 1) return cd;
                return cd + " * (" + idx() + ")S" + std::to_string(L) + "_" + std::to_string(d);
            }

            // Emit coordinates c<d> for `dims` (row-major) from index `var`.
            void decompose(std::ostringstream& o, const std::string& ind, const std::string& var, const std::vector<int>& dims) {
                if (dims.empty()) return;
                const std::string t = idx();
                o << ind << "{ " << t << " rem_ = " << var << ";\n";
                // One scope per dim: each step declares its own quotient.
                for (size_t k = dims.size() - 1; k >= 1; --k) {
                    const std::string d = std::to_string(dims[k]);
                    if (idx32)
                        o << ind << "  { const " << t << " q_ = (" << t << ")ormi_fdiv((unsigned)rem_, (unsigned)M" << d
                          << ", (unsigned)(M" << d << " >> 32));";
                    else
                        o << ind << "  { const long long q_ = rem_ / D" << d << ";";
                    o << " c" << d << " = rem_ - q_ * (" << t << ")D" << d << "; rem_ = q_; }\n";
                }
                o << ind << "  c" << dims[0] << " = rem_; }\n";
                for (int d : dims)
                    if (d == vec_dim && vec > 1) o << ind << "c" << d << " *= " << vec << ";\n";
            }

            void declare_coords(std::ostringstream& o, const std::string& ind, const std::vector<int>& dims) {
                for (int d : dims) o << ind << idx() << " c" << d << " = 0;\n";
            }

            // Offset expression of leaf L over `dims`, empty when all terms vanish.
            std::string offset(size_t L, const std::vector<int>& dims) const {
                std::string s;
                for (int d : dims) {
                    std::string t = stride_term(L, d);
                    if (t.empty()) continue;
                    s += s.empty() ? t : " + " + t;
                }
                return s;
            }

            // Load leaf L at element offset `off` into dst[0..vec).
            void load_leaf(std::ostringstream& o, const std::string& ind, size_t L, const std::string& off, const std::string& dst) {
                const DType dt = e.leaves[L].dtype;
                const std::string p = "L" + std::to_string(L);
                if (scalar[L]) return;  // hoisted
                const bool unit = vec > 1 && c.st[L][vec_dim] == 1;
                const bool nt = nt_loads && streamed(L);
                if (unit) {
                    const char* vt = dt == DType::Float32 ? "ormi_f4" : "ormi_u16x4";
                    const std::string addr = elem_ptr(std::string("const ") + vt + "*", p, off, dtype_size(dt), true);
                    o << ind << "{ const " << vt << " v_ = " << (nt ? "__builtin_nontemporal_load(" + addr + ")" : "*" + addr) << ";";
                    for (int k = 0; k < vec; ++k) {
                        const std::string ek = "v_[" + std::to_string(k) + "]";
                        o << " " << dst << "[" << k << "] = " << (dt == DType::Float32 ? ek : to_f32(dt, ek)) << ";";
                    }
                    o << " }\n";
                } else {
                    const std::string elem = off32 ? "*" + elem_ptr(std::string("const ") + storage_type(dt) + "*", p, off,
                                                                    dtype_size(dt), true)
                                                   : p + "[" + off + "]";
                    o << ind << "{ const float v_ = " << to_f32(dt, elem) << ";";
                    for (int k = 0; k < vec; ++k) o << " " << dst << "[" << k << "] = v_;";
                    o << " }\n";
                }
            }

            void hoist_scalars(std::ostringstream& o, const std::string& ind) {
                for (size_t L = 0; L < e.leaves.size(); ++L)
                    if (scalar[L])
                        o << ind << "const float s" << L << " = " << to_f32(e.leaves[L].dtype, "L" + std::to_string(L) + "[0]") << ";\n";
            }

            // Value names of expr.roots after the last eval().
            std::vector<std::string> root_names;

            // SSA evaluation for vector element k: leaf values come from
            // x<L>[u][k] (or the hoisted scalar). Returns the root value name.
            std::string eval(std::ostringstream& o, const std::string& ind, const std::string& u, const std::string& k) {
                std::vector<std::string> name(e.leaves.size() + e.insts.size());
                for (size_t L = 0; L < e.leaves.size(); ++L)
                    name[L] = scalar[L] ? "s" + std::to_string(L) : "x" + std::to_string(L) + "[" + u + "][" + k + "]";
                for (size_t i = 0; i < e.insts.size(); ++i) {
                    const Inst& in = e.insts[i];
                    const size_t id = e.leaves.size() + i;
                    std::string expr;
                    if (in.op == OpEnum::CAST) {
                        if (in.cast == DType::BFloat16) expr = "ormi_round_bf16(" + name[in.a] + ")";
                        else if (in.cast == DType::Float16) expr = "ormi_round_f16(" + name[in.a] + ")";
                        else expr = name[in.a];
                    } else {
                        std::vector<std::string> operands{name[in.a]};
                        if (in.b >= 0) operands.push_back(name[in.b]);
                        if (!in.lower)
                            throw std::runtime_error(std::string("HIP JIT Compiler Error: No lowering rule registered for ") +
                                                     ops::op_name(in.op));
                        expr = (*in.lower)(operands);
                    }
                    name[id] = "t" + std::to_string(i);
                    o << ind << "const float " << name[id] << " = " << expr << ";\n";
                }
                root_names.clear();
                for (int r : e.roots) root_names.push_back(name[r]);
                return name[e.root];
            }

            // Registers x<L>[unroll][vec] of every non-scalar leaf whose `pick` entry
            // is true (all of them when pick is empty).
            void declare_leaf_regs(std::ostringstream& o, const std::string& ind, int unroll,
                                   const std::vector<bool>& pick = {}) {
                for (size_t L = 0; L < e.leaves.size(); ++L)
                    if (!scalar[L] && (pick.empty() || pick[L]))
                        o << ind << "float x" << L << "[" << unroll << "][" << vec << "];\n";
            }

            std::string finish(const std::string& kind, int block, KernelLaunch& k) {
                std::ostringstream sig;
                for (size_t i = 0; i < args.decls.size(); ++i) sig << (i ? ",\n    " : "    ") << render(args.decls[i]);
                const std::string kernel_body = body().str();
                k.name = "ormi_" + kind + "_" + hex_hash(kernel_body + sig.str());
                std::ostringstream src;
                src << kDeviceHeader << "\n\nextern \"C\" __global__ __launch_bounds__(" << block << ") void " << k.name << "(\n"
                    << sig.str() << ") {\n" << kernel_body << "}\n";
                return src.str();
            }
        };

        std::vector<int> dims_of(const Canon& c, Group g) {
            std::vector<int> v;
            for (size_t d = 0; d < c.dims.size(); ++d)
                if (c.dims[d].group == g) v.push_back((int)d);
            return v;
        }

        long long group_size(const Canon& c, Group g) {
            long long n = 1;
            for (auto& d : c.dims)
                if (d.group == g) n *= d.size;
            return n;
        }

        const Expr& no_expr() {
            static const Expr e;
            return e;
        }

        const char* reduce_name(ReduceOp op) {
            return op == ReduceOp::Sum ? "sum" : op == ReduceOp::Max ? "max" : "argmax";
        }

        // ------------------------------------------------ store epilogue --
        // Kernel arguments of a store epilogue: its output (epo) and its
        // scalar operands (E<leaf>), read once per stored element.
        void declare_epilogue(Gen& g, const StoreEpilogue* ep) {
            if (!ep) return;
            g.args.ptr(false, storage_type(ep->out_dtype), "epo", ep->out);
            for (size_t L = 0; L < ep->expr.leaves.size(); ++L)
                if ((int)L != ep->value)
                    g.args.ptr(true, storage_type(ep->expr.leaves[L].dtype), "E", ep->expr.leaves[L].ptr, (int)L);
        }

        // Statements that evaluate the epilogue of the reduced value `v` and
        // store it at element `at` of epo. The tape is lowered exactly as a
        // map kernel lowers it, so the stored bits equal those of the
        // element-wise kernel it replaces.
        void emit_epilogue(std::ostringstream& b, const std::string& ind, const StoreEpilogue* ep, const std::string& v,
                           const std::string& at) {
            if (!ep) return;
            const Expr& e = ep->expr;
            std::vector<std::string> name(e.leaves.size() + e.insts.size());
            b << ind << "{\n";
            for (size_t L = 0; L < e.leaves.size(); ++L) {
                name[L] = "ev" + std::to_string(L);
                const std::string src = (int)L == ep->value ? v : to_f32(e.leaves[L].dtype, "E" + std::to_string(L) + "[0]");
                b << ind << "  const float " << name[L] << " = " << src << ";\n";
            }
            for (size_t i = 0; i < e.insts.size(); ++i) {
                const Inst& in = e.insts[i];
                std::string expr;
                if (in.op == OpEnum::CAST) {
                    if (in.cast == DType::BFloat16) expr = "ormi_round_bf16(" + name[in.a] + ")";
                    else if (in.cast == DType::Float16) expr = "ormi_round_f16(" + name[in.a] + ")";
                    else expr = name[in.a];
                } else {
                    std::vector<std::string> operands{name[in.a]};
                    if (in.b >= 0) operands.push_back(name[in.b]);
                    if (!in.lower) throw std::runtime_error(std::string("HIP JIT Compiler Error: No lowering rule registered for ") +
                                                            ops::op_name(in.op));
                    expr = (*in.lower)(operands);
                }
                name[e.leaves.size() + i] = "et" + std::to_string(i);
                b << ind << "  const float et" << i << " = " << expr << ";\n";
            }
            b << ind << "  epo[" << at << "] = " << from_f32(ep->out_dtype, name[e.root]) << ";\n" << ind << "}\n";
        }

        // Signature part of a store epilogue (its arguments are in the
        // declarations already).
        std::string epilogue_layout(const StoreEpilogue* ep) {
            if (!ep) return std::string();
            std::string s = "|ep";
            append_int(s, ep->value);
            s += ',';
            s += char('a' + (int)ep->out_dtype);
            for (const Leaf& L : ep->expr.leaves) s += char('a' + (int)L.dtype);
            for (const Inst& in : ep->expr.insts) {
                s += ';';
                append_int(s, (int)in.op);
                s += ',';
                append_int(s, in.a);
                s += ',';
                append_int(s, in.b);
                s += ',';
                append_int(s, (int)in.cast);
            }
            s += ';';
            append_int(s, ep->expr.root);
            return s;
        }

        void check_epilogue(const StoreEpilogue* ep, ReduceOp op) {
            if (!ep) return;
            if (op == ReduceOp::Argmax) throw std::runtime_error("HIP reduce: no store epilogue on an argmax.");
            const Expr& e = ep->expr;
            if (ep->value < 0 || ep->value >= (int)e.leaves.size() || e.root < 0 ||
                e.root >= (int)(e.leaves.size() + e.insts.size()) || !ep->out)
                throw std::runtime_error("HIP reduce: malformed store epilogue.");
            for (size_t L = 0; L < e.leaves.size(); ++L)
                if ((int)L != ep->value && !e.leaves[L].scalar)
                    throw std::runtime_error("HIP reduce: store epilogue operands must be scalars.");
        }

        // Everything a generated source depends on, without sizes, strides or
        // pointers: kernel kind, parameter list, which strides are 0 / 1 /
        // general, group layout, vector width, index width, tuning and the tape.
        std::string signature(const Gen& g, const std::string& kind) {
            std::string s;
            s.reserve(256);
            const Tuning& t = tuning();
            s += kind;
            s += '|';
            for (long long v : {(long long)t.map_unroll, (long long)t.row_unroll, (long long)t.col_waves, (long long)t.row_waves,
                                (long long)t.row_waves_min_groups, (long long)t.col_unroll, (long long)t.col_fin_split}) {
                append_int(s, v);
                s += ',';
            }
            s += char('0' + g.nt_loads);
            s += char('0' + t.map_nt_stores);
            s += '|';
            for (const auto& d : g.args.decls) {
                s += d.is_const ? 'c' : 'm';
                s += d.type;
                s += d.is_ptr ? '*' : ' ';
                s += d.name;
                append_int(s, d.i);
                s += '_';
                append_int(s, d.j);
                s += ';';
            }
            // Element types, which the storage types above do not fix: bf16
            // and fp16 are both unsigned short, but load and store differently.
            s += '|';
            for (const auto& L : g.e.leaves) s += char('a' + (int)L.dtype);
            s += '/';
            for (DType dt : g.out_dtypes) s += char('a' + (int)dt);
            s += '|';
            for (const auto& d : g.c.dims) s += char('0' + (int)d.group);
            s += '|';
            append_int(s, g.vec);
            s += ',';
            append_int(s, g.vec_dim);
            s += g.off32 ? ",32u," : g.idx32 ? ",32," : ",64,";
            append_int(s, g.rows);
            s += '|';
            for (size_t L = 0; L < g.e.leaves.size(); ++L) {
                if (g.scalar[L]) {
                    s += 'S';
                    continue;
                }
                for (long long v : g.c.st[L]) s += v == 0 ? '0' : v == 1 ? '1' : 'x';
                s += ',';
            }
            s += '|';
            for (const auto& in : g.e.insts) {
                append_int(s, (int)in.op);
                s += ',';
                append_int(s, in.a);
                s += ',';
                append_int(s, in.b);
                s += ',';
                append_int(s, (int)in.cast);
                s += ';';
            }
            append_int(s, g.e.root);
            for (int r : g.e.roots) {
                s += ',';
                append_int(s, r);
            }
            return s;
        }

        // Generated kernels by signature: name and source once emitted, and
        // the hipRTC handle once compiled.
        struct CachedKernel {
            std::string name;
            std::string source;
            uint64_t handle = 0;
        };
        std::mutex& cache_mu() {
            static std::mutex m;
            return m;
        }
        std::unordered_map<std::string, CachedKernel>& kernel_cache() {
            static auto* c = new std::unordered_map<std::string, CachedKernel>();
            return *c;
        }

        // On a hit, fills k's name and handle (or source) and returns true.
        bool cache_lookup(const std::string& sig, KernelLaunch& k) {
            k.key = sig;
            std::lock_guard<std::mutex> lock(cache_mu());
            auto it = kernel_cache().find(sig);
            if (it == kernel_cache().end()) return false;
            k.name = it->second.name;
            k.handle = it->second.handle;
            if (!k.handle) k.source = it->second.source;
            return true;
        }

        void cache_store(const KernelLaunch& k) {
            std::lock_guard<std::mutex> lock(cache_mu());
            auto& e = kernel_cache()[k.key];
            e.name = k.name;
            if (!k.source.empty()) e.source = k.source;
            if (k.handle) e.handle = k.handle;
        }

        // Emit the source of a kernel unless the cache already has it.
        // layout: whatever else the emitted body depends on that the signature
        // does not see (a column kernel's waves across columns, which follow
        // the kept extent). The block size is part of the key too.
        template <typename EmitBody>
        void resolve(Gen& g, const std::string& kind, int block, KernelLaunch& k, EmitBody emit,
                     const std::string& layout = std::string()) {
            k.args = g.args.vals;
            k.block[0] = (uint32_t)block;
            k.ptr_slots.clear();
            for (size_t i = 0; i < g.args.decls.size(); ++i) {
                const ArgDecl& d = g.args.decls[i];
                if (!d.is_ptr) continue;
                const std::string_view name(d.name);
                if (name == "L") k.ptr_slots.push_back({(int)i, d.i});
                else if (name == "out") k.ptr_slots.push_back({(int)i, -1 - std::max(d.i, 0)});
                else if (name == "outp" && g.args.vals[i] != 0) k.ptr_slots.push_back({(int)i, -1});
                else if (name == "epo") k.ptr_slots.push_back({(int)i, -2});
                else if (name == "E") k.ptr_slots.push_back({(int)i, kEpilogueLeaf + d.i});
            }
            std::string sig = signature(g, kind);
            sig += "|b";
            append_int(sig, block);
            sig += layout;
            if (cache_lookup(sig, k)) return;
            emit();
            k.source = g.finish(kind, block, k);
            cache_store(k);
        }
    }  // namespace

    std::string kernel_source(const KernelLaunch& k) {
        if (!k.source.empty() || k.key.empty()) return k.source;
        std::lock_guard<std::mutex> lock(cache_mu());
        auto it = kernel_cache().find(k.key);
        return it == kernel_cache().end() ? std::string() : it->second.source;
    }

    std::string PlanInfo::text() const {
        std::string s = kind;
        if (op) {
            s += ' ';
            s += op;
        }
        for (int i = 0; i < n; ++i) {
            s += ' ';
            s += field[i].first;
            s += '=';
            s += std::to_string(field[i].second);
        }
        return s;
    }

    // ------------------------------------------------------------------ map --
    static KernelLaunch plan_map_multi_uncached(const Expr& expr, const std::vector<int>& shape, const std::vector<void*>& outs,
                                                const std::vector<DType>& out_dtypes, int cu) {
        if (outs.size() != expr.roots.size() || outs.size() != out_dtypes.size() || outs.empty())
            throw std::runtime_error("HIP codegen: one output buffer and dtype per root.");
        const size_t nout = outs.size();
        const Tuning& tn = tuning();
        const int block = 256, unroll = tn.map_unroll;
        Gen g(expr);
        g.out_dtypes = out_dtypes;
        g.want_off32 = tn.map_off32;
        for (int s : shape) g.c.dims.push_back({(long long)s, G_M});
        for (const auto& L : expr.leaves) g.c.st.push_back(L.st);
        canonicalize(g.c, g.scalar);
        if (g.c.dims.empty()) {
            g.c.dims.push_back({1, G_M});
            for (auto& s : g.c.st) s.push_back(0);
        }
        const int n = (int)g.c.dims.size();
        g.choose_vec(n - 1);
        for (size_t r = 0; r < nout; ++r)
            if (!vector_dtype(out_dtypes[r]) || ((uintptr_t)outs[r] % 16) != 0) g.vec = 1;
        long long numel = 1;
        for (auto& d : g.c.dims) numel *= d.size;
        g.choose_nt_loads(tn.map_nt_loads, numel);
        const long long G = numel / g.vec;
        const long long tile = (long long)block * unroll;
        const long long tiles = (G + tile - 1) / tile;
        long long grid = std::max(1LL, std::min(tiles, (long long)std::max(cu, 1) * tn.map_blocks_per_cu));
        // The grid-stride cursor reaches G + grid * tile before the loop exits.
        int out_bytes = 1;
        for (DType dt : out_dtypes) out_bytes = std::max(out_bytes, (int)dtype_size(dt));
        g.choose_idx(G + grid * tile, out_bytes);

        // Tiles aligned to the last dim, which holds Dl groups (32-bit indices,
        // two or more dims):
        //  rows 1: a tile covers P = tile / Dl > 1 whole rows. Each lane keeps its
        //          last-dim coordinate and its row within the tile for the whole
        //          loop: operands that vary only along the last dim are loaded once
        //          before the loop, and an access's row is the tile's first row
        //          plus that lane constant (no division per element);
        //  rows 2: a tile lies inside one row (Dl a multiple of tile). The outer
        //          coordinates are uniform per tile, so they and the loads of
        //          operands that vary only across rows are scalar work, and every
        //          tile is full, so stores need no bounds guard;
        //  rows 3: a tile is exactly one row (tile == Dl): both of the above;
        //  rows 4: rows 2 where operands vary only along the last dim (a bias
        //          row): a tile is `unroll` consecutive rows of one 256-group
        //          window (NW = Dl / 256 windows per row), so each lane loads those
        //          operands once for all its rows. The grid is a multiple of NW,
        //          so a block keeps its window and loads them once per block.
        const int n_last = n - 1;
        const long long Dl = g.c.dims[n_last].size / g.vec;
        if (tn.map_rows && g.idx32 && n >= 2 && Dl > 0) {
            if (tile == Dl) g.rows = 3;
            else if (tile % Dl == 0) g.rows = 1;
            else if (Dl % tile == 0) g.rows = 2;
        }
        // Leaves that vary only along the last dim: zero stride on every outer dim.
        std::vector<bool> only_last(expr.leaves.size(), false);
        bool any_only_last = false;
        for (size_t L = 0; L < expr.leaves.size(); ++L) {
            if (g.scalar[L]) continue;
            bool o = true;
            for (int d = 0; d < n_last; ++d) o = o && g.c.st[L][d] == 0;
            only_last[L] = o;
            any_only_last = any_only_last || o;
        }
        long long NW = 0;
        const long long R = Dl > 0 ? G / Dl : 0;
        if (g.rows == 2 && any_only_last && tn.map_row_tiles && unroll > 1 && R % unroll == 0) {
            NW = Dl / block;
            const long long gr = grid / NW * NW;
            if (gr >= NW) {
                g.rows = 4;
                grid = gr;
            }
        }
        const int rows = g.rows;
        // Leaves loaded once before the loop (rows 1, 3 and 4).
        std::vector<bool> hoist(expr.leaves.size(), false), in_loop(expr.leaves.size(), true);
        if (rows == 1 || rows == 3 || rows == 4)
            for (size_t L = 0; L < expr.leaves.size(); ++L) {
                if (g.scalar[L]) continue;
                hoist[L] = only_last[L];
                in_loop[L] = !only_last[L];
            }

        // A single output keeps the name "out"; several are out0, out1, ...
        auto out_name = [&](size_t r) { return nout == 1 ? std::string("out") : "out" + std::to_string(r); };
        KernelLaunch k;
        for (size_t r = 0; r < nout; ++r)
            g.args.ptr(false, storage_type(out_dtypes[r]), "out", outs[r], nout == 1 ? -1 : (int)r);
        g.declare_leaves();
        g.args.i64("G", G);
        g.declare_dims();
        g.declare_strides();
        if (rows == 1) {
            g.args.i64("R", G / Dl);
            g.args.i64("P", tile / Dl);
        }
        if (rows == 4) {
            g.args.i64("R", R);
            g.args.i64("NW", NW);
        }
        k.grid[0] = (uint32_t)grid;
        // The cap pays where the kernel writes about as much as it reads (a
        // copy, C2); a kernel that mostly reads keeps every slot (the capped
        // read-only kernels of the ceiling probe ran slower). Tiles of several
        // rows take one more work-group per CU: C2 on them ran 43.6-43.9 us at
        // 6, 44.2-44.6 at 5 and 44.2-44.4 at 7, against 44.0-44.1 on one-row
        // tiles at 5 (44.3-44.6 at 6).
        long long write_bytes = 0;
        for (DType dt : out_dtypes) write_bytes += (long long)dtype_size(dt);
        if (2 * write_bytes >= g.streamed_bytes(1))
            k.lds = occupancy_lds(rows == 4 ? tn.map_row_tile_wg_per_cu : tn.map_wg_per_cu, grid, cu);
        k.plan.kind = "map";
        k.plan.add("ndim", n);
        k.plan.add("vec", g.vec);
        k.plan.add("idx", g.idx32 ? 32 : 64);
        k.plan.add("off32", g.off32 ? 1 : 0);
        k.plan.add("rows", rows);
        k.plan.add("groups", G);
        k.plan.add("unroll", unroll);
        if (k.lds) k.plan.add("lds", k.lds);
        if (nout > 1) k.plan.add("outputs", (long long)nout);
        resolve(g, "map", block, k, [&] {
            std::vector<int> all, outer;
            for (int d = 0; d < n; ++d) all.push_back(d);
            for (int d = 0; d < n_last; ++d) outer.push_back(d);
            const std::string t = g.idx();
            const std::string tid = "(" + t + ")threadIdx.x";
            const std::string lane = "u * " + std::to_string(block) + " + " + tid;  // group offset within the tile
            const std::string cl = "c" + std::to_string(n_last);
            const std::string Dn = "D" + std::to_string(n_last), Mn = "M" + std::to_string(n_last);
            const int V = g.vec;
            std::ostringstream& b = g.body();
            auto load_all = [&](const std::string& ind, const std::vector<bool>& pick) {
                for (size_t L = 0; L < expr.leaves.size(); ++L) {
                    if (g.scalar[L] || !pick[L]) continue;
                    std::string off = g.offset(L, all);
                    g.load_leaf(b, ind, L, off.empty() ? "0" : off, "x" + std::to_string(L) + "[u]");
                }
            };
            g.hoist_scalars(b, "  ");
            b << "  const " << t << " tile = " << tile << ";\n";
            if (rows == 1 || rows == 3) {
                // Per-lane constants: last-dim coordinate (times VEC) and, for
                // rows 1, the row within the tile.
                b << "  " << t << " cl_[" << unroll << "];\n";
                if (rows == 1) b << "  " << t << " q_[" << unroll << "];\n";
                b << "#pragma unroll\n  for (int u = 0; u < " << unroll << "; ++u) {\n";
                b << "    const " << t << " l_ = " << lane << ";\n";
                if (rows == 1) {
                    b << "    const " << t << " q = (" << t << ")ormi_fdiv((unsigned)l_, (unsigned)" << Mn << ", (unsigned)(" << Mn
                      << " >> 32));\n";
                    b << "    q_[u] = q;\n    cl_[u] = (l_ - q * (" << t << ")" << Dn << ") * " << V << ";\n";
                } else {
                    b << "    cl_[u] = l_ * " << V << ";\n";
                }
                b << "  }\n";
                g.declare_leaf_regs(b, "  ", unroll, hoist);
                b << "#pragma unroll\n  for (int u = 0; u < " << unroll << "; ++u) {\n";
                b << "    const " << t << " " << cl << " = cl_[u];\n";
                load_all("    ", hoist);
                b << "  }\n";
                const std::string step = rows == 1 ? "(" + t + ")P" : "1";
                b << "  for (" << t << " base = (" << t << ")blockIdx.x * tile, row = (" << t << ")blockIdx.x * " << step
                  << "; base < (" << t << ")G; base += (" << t << ")gridDim.x * tile, row += (" << t << ")gridDim.x * " << step
                  << ") {\n";
                g.declare_leaf_regs(b, "    ", unroll, in_loop);
                if (rows == 3) {
                    g.declare_coords(b, "    ", outer);
                    g.decompose(b, "    ", "row", outer);
                }
                b << "#pragma unroll\n    for (int u = 0; u < " << unroll << "; ++u) {\n";
                if (rows == 1) {
                    // The last tile may hold fewer than P rows: clamp the row for the loads.
                    b << "      const " << t << " o_ = row + q_[u] < (" << t << ")R ? row + q_[u] : (" << t << ")R - 1;\n";
                    g.declare_coords(b, "      ", outer);
                    g.decompose(b, "      ", "o_", outer);
                }
                b << "      const " << t << " " << cl << " = cl_[u];\n";
                load_all("      ", in_loop);
                b << "    }\n";
            } else if (rows == 2) {
                b << "  for (" << t << " base = (" << t << ")blockIdx.x * tile; base < (" << t << ")G; base += (" << t
                  << ")gridDim.x * tile) {\n";
                b << "    const " << t << " row = (" << t << ")ormi_fdiv((unsigned)base, (unsigned)" << Mn << ", (unsigned)(" << Mn
                  << " >> 32));\n";
                b << "    const " << t << " col0 = base - row * (" << t << ")" << Dn << ";\n";
                g.declare_coords(b, "    ", outer);
                g.decompose(b, "    ", "row", outer);
                g.declare_leaf_regs(b, "    ", unroll);
                b << "#pragma unroll\n    for (int u = 0; u < " << unroll << "; ++u) {\n";
                b << "      const " << t << " " << cl << " = (col0 + " << lane << ") * " << V << ";\n";
                load_all("      ", in_loop);
                b << "    }\n";
            } else if (rows == 4) {
                // The grid is a multiple of NW, so a block's window (blockIdx.x
                // mod NW) is the same in every tile it visits; its rows advance
                // by gridDim.x / NW tiles of `unroll` rows.
                b << "  const " << t << " col0 = ((" << t << ")blockIdx.x % (" << t << ")NW) * " << block << ";\n";
                b << "  const " << t << " " << cl << " = (col0 + " << tid << ") * " << V << ";\n";
                g.declare_leaf_regs(b, "  ", unroll, hoist);
                b << "  {\n    const int u = 0;\n";
                load_all("    ", hoist);
                b << "  }\n";
                for (size_t L = 0; L < expr.leaves.size(); ++L)
                    if (hoist[L])
                        b << "#pragma unroll\n  for (int u = 1; u < " << unroll << "; ++u)\n#pragma unroll\n    for (int k = 0; k < "
                          << V << "; ++k) x" << L << "[u][k] = x" << L << "[0][k];\n";
                b << "  for (" << t << " row0 = (" << t << ")blockIdx.x / (" << t << ")NW * " << unroll << "; row0 < (" << t
                  << ")R; row0 += (" << t << ")gridDim.x / (" << t << ")NW * " << unroll << ") {\n";
                g.declare_leaf_regs(b, "    ", unroll, in_loop);
                b << "#pragma unroll\n    for (int u = 0; u < " << unroll << "; ++u) {\n";
                b << "      const " << t << " row = row0 + u;\n";
                g.declare_coords(b, "      ", outer);
                g.decompose(b, "      ", "row", outer);
                load_all("      ", in_loop);
                b << "    }\n";
            } else {
                b << "  for (" << t << " base = (" << t << ")blockIdx.x * tile; base < (" << t << ")G; base += (" << t
                  << ")gridDim.x * tile) {\n";
                g.declare_leaf_regs(b, "    ", unroll);
                b << "#pragma unroll\n    for (int u = 0; u < " << unroll << "; ++u) {\n";
                b << "      const " << t << " gg = base + " << lane << ";\n";
                b << "      const " << t << " gc = gg < (" << t << ")G ? gg : (" << t << ")G - 1;\n";
                g.declare_coords(b, "      ", all);
                g.decompose(b, "      ", "gc", all);
                load_all("      ", in_loop);
                b << "    }\n";
            }
            // rows 2 and 3 tiles are always full; rows 0 and 1 guard the last one.
            const bool guard = rows == 0 || rows == 1;
            b << "#pragma unroll\n    for (int u = 0; u < " << unroll << "; ++u) {\n";
            auto res = [&](size_t r) { return nout == 1 ? std::string("res") : "res" + std::to_string(r); };
            for (size_t r = 0; r < nout; ++r) b << "      float " << res(r) << "[" << V << "];\n";
            b << "#pragma unroll\n      for (int k = 0; k < " << V << "; ++k) {\n";
            g.eval(b, "        ", "u", "k");
            for (size_t r = 0; r < nout; ++r) b << "        " << res(r) << "[k] = " << g.root_names[r] << ";\n";
            b << "      }\n";
            if (rows == 4) b << "      const " << t << " go = (row0 + u) * (" << t << ")" << Dn << " + col0 + " << tid << ";\n";
            else b << "      const " << t << " go = base + " << lane << ";\n";
            if (guard) b << "      if (go < (" << t << ")G) {\n";
            const std::string ind = guard ? "        " : "      ";
            const bool nt = tn.map_nt_stores;
            for (size_t r = 0; r < nout; ++r) {
                const DType odt = out_dtypes[r];
                if (V == 4) {
                    const char* vt = odt == DType::Float32 ? "ormi_f4" : "ormi_u16x4";
                    std::string val = std::string(vt) + "{";
                    for (int q = 0; q < 4; ++q) val += (q ? ", " : "") + from_f32(odt, res(r) + "[" + std::to_string(q) + "]");
                    val += "}";
                    const std::string addr = g.elem_ptr(std::string(vt) + "*", out_name(r), "go * 4", dtype_size(odt), false);
                    if (nt) b << ind << "__builtin_nontemporal_store(" << val << ", " << addr << ");\n";
                    else b << ind << "*" << addr << " = " << val << ";\n";
                } else {
                    b << ind << "*" << g.elem_ptr(std::string(storage_type(odt)) + "*", out_name(r), "go", dtype_size(odt), false)
                      << " = " << from_f32(odt, res(r) + "[0]") << ";\n";
                }
            }
            if (guard) b << "      }\n";
            b << "    }\n  }\n";
        });
        return k;
    }

    // ------------------------------------------------------------- reduce --
    static ReducePlan plan_reduce_uncached(const Expr& expr, const std::vector<int>& in_shape, const std::vector<int>& axes_in,
                                           ReduceOp op, void* out, int cu, const StoreEpilogue* ep) {
        check_epilogue(ep, op);
        const std::string ep_layout = epilogue_layout(ep);
        const Tuning& tn = tuning();
        const int n = (int)in_shape.size();
        std::vector<bool> red(n, axes_in.empty());
        for (int a : axes_in) red[a] = true;
        int last_red = -1;
        for (int d = 0; d < n; ++d)
            if (red[d]) last_red = d;

        Gen g(expr);
        // Kernel dim order: O dims, R dims, I dims (each in logical order).
        std::vector<int> perm;
        for (int d = 0; d < n; ++d) if (!red[d] && d < last_red) perm.push_back(d);
        for (int d = 0; d < n; ++d) if (red[d]) perm.push_back(d);
        for (int d = 0; d < n; ++d) if (!red[d] && d > last_red) perm.push_back(d);
        for (int d : perm) g.c.dims.push_back({(long long)in_shape[d], red[d] ? G_R : (d < last_red ? G_O : G_I)});
        for (const auto& L : expr.leaves) {
            std::vector<long long> s;
            for (int d : perm) s.push_back(L.st[d]);
            g.c.st.push_back(s);
        }
        canonicalize(g.c, g.scalar);

        const long long O = group_size(g.c, G_O), R = group_size(g.c, G_R), I = group_size(g.c, G_I);
        g.choose_nt_loads(tn.reduce_nt_loads, O * R * I);
        if (R >= (1ll << 31)) throw std::runtime_error("HIP reduce: reduced extent above 2^31 elements.");
        const std::vector<int> od = dims_of(g.c, G_O), rd = dims_of(g.c, G_R), id = dims_of(g.c, G_I);
        const bool column = !id.empty();
        g.choose_vec(column ? id.back() : (rd.empty() ? -1 : rd.back()));

        ReducePlan plan;
        KernelLaunch& k = plan.first;
        const char* name = reduce_name(op);
        const bool is_sum = op == ReduceOp::Sum;
        const bool is_arg = op == ReduceOp::Argmax;
        const int V = g.vec;

        if (!column) {
            // ---------------------------------------------------------- row --
            const int RU = tn.row_unroll;
            const long long RG = R / V;
            long long P = 1;
            const long long target_waves = (long long)std::max(cu, 1) * 32;
            if (O < target_waves / 2) P = std::max(1LL, std::min((target_waves + O - 1) / O, (RG + 255) / 256));
            const long long CH = (RG + P - 1) / P;
            P = RG == 0 ? 1 : (RG + CH - 1) / CH;  // drop empty parts
            g.choose_idx(O * P * 64 + RG * V + 64 * V * RU);
            plan.two_pass = P > 1;
            // Long rows that need no split: WR waves of one block share a row
            // and combine their results through LDS in wave order. Shorter
            // waves leave a shorter tail when the grid drains (C3's 32 KB
            // rows: 78.4 us with four waves per row against 81.6 with one,
            // the same reads).
            const int WR = (P == 1 && CH >= tn.row_waves_min_groups) ? tn.row_waves : 1;
            const StoreEpilogue* ep1 = plan.two_pass ? nullptr : ep;  // the finishing kernel stores a split result
            g.args.ptr(false, "void", "outp", plan.two_pass ? nullptr : out);  // workspace bound later
            g.args.ptr(false, "int", "outi", nullptr);
            g.declare_leaves();
            declare_epilogue(g, ep1);
            g.args.i64("NO", O);
            g.args.i64("NP", P);
            g.args.i64("RG", RG);
            g.args.i64("CH", CH);
            g.declare_dims();
            g.declare_strides();
            const int UPB = 4 / WR;  // (row, part) units per 256-thread block
            k.grid[0] = (uint32_t)std::max(1LL, (O * P + UPB - 1) / UPB);
            // Shared rows only (long-lived work-groups of 32 KB of reads and more;
            // the cap starves short-lived ones, as in the ceiling probe).
            if (WR > 1) k.lds = occupancy_lds(is_sum ? tn.row_wg_per_cu : tn.row_max_wg_per_cu, k.grid[0], cu);
            k.plan.kind = "row";
            k.plan.op = name;
            for (auto [key, v] : {std::pair<const char*, long long>{"O", O}, {"R", R}, {"vec", V}, {"parts", P},
                                  {"waves_per_row", WR}, {"idx", g.idx32 ? 32 : 64}})
                k.plan.add(key, v);
            if (k.lds) k.plan.add("lds", k.lds);
            resolve(g, std::string("row") + name + (WR > 1 ? "_w" + std::to_string(WR) : std::string()), 256, k, [&] {
                const std::string t = g.idx();
                std::ostringstream& b = g.body();
                g.hoist_scalars(b, "  ");
                b << "  const int lane = threadIdx.x & 63;\n";
                if (WR == 1) {
                    b << "  const " << t << " wid = (" << t << ")blockIdx.x * 4 + (" << t << ")(threadIdx.x >> 6);\n";
                    b << "  if (wid >= (" << t << ")NO * (" << t << ")NP) return;\n";
                } else {
                    // Every wave reaches the barrier below; a wave past the last
                    // unit reads unit 0's row and its result is dropped.
                    b << "  const int wv = (int)(threadIdx.x >> 6), q = wv % " << WR << ";\n";
                    b << "  const " << t << " wid_ = (" << t << ")blockIdx.x * " << UPB << " + (" << t << ")(wv / " << WR << ");\n";
                    b << "  const bool live = wid_ < (" << t << ")NO * (" << t << ")NP;\n";
                    b << "  const " << t << " wid = live ? wid_ : 0;\n";
                }
                b << "  const " << t << " o = wid / (" << t << ")NP, p = wid - o * (" << t << ")NP;\n";
                g.declare_coords(b, "  ", od);
                g.decompose(b, "  ", "o", od);
                for (size_t L = 0; L < expr.leaves.size(); ++L) {
                    if (g.scalar[L]) continue;
                    std::string off = g.offset(L, od);
                    b << "  const " << t << " base" << L << " = " << (off.empty() ? "0" : off) << ";\n";
                }
                if (WR == 1) {
                    b << "  const " << t << " rg0 = p * (" << t << ")CH;\n";
                    b << "  const " << t << " rg1 = rg0 + (" << t << ")CH < (" << t << ")RG ? rg0 + (" << t << ")CH : (" << t << ")RG;\n";
                } else {
                    // Wave q takes the q-th of WR consecutive pieces of the part, each a
                    // whole number of 64-group strides.
                    b << "  const " << t << " pr0 = p * (" << t << ")CH;\n";
                    b << "  const " << t << " pr1 = pr0 + (" << t << ")CH < (" << t << ")RG ? pr0 + (" << t << ")CH : (" << t << ")RG;\n";
                    b << "  const " << t << " sc = ((pr1 - pr0 + " << WR - 1 << ") / " << WR << " + 63) / 64 * 64;\n";
                    b << "  const " << t << " rg0 = pr0 + q * sc < pr1 ? pr0 + q * sc : pr1;\n";
                    b << "  const " << t << " rg1 = rg0 + sc < pr1 ? rg0 + sc : pr1;\n";
                }
                if (is_sum) b << "  float acc[" << V << "];\n#pragma unroll\n  for (int k = 0; k < " << V << "; ++k) acc[k] = 0.0f;\n";
                // max / argmax: one (value, index) chain per vector slot, so
                // the V chains advance independently.
                else b << "  float mv[" << V << "]; int mi[" << V << "];\n#pragma unroll\n  for (int k = 0; k < " << V
                       << "; ++k) { mv[k] = -__builtin_inff(); mi[k] = 0x7fffffff; }\n";
                // UNR groups per lane starting at rg, 64 groups apart.
                auto emit_step = [&](int UNR, const std::string& ind) {
                    g.declare_leaf_regs(b, ind, UNR);
                    b << ind << "#pragma unroll\n" << ind << "for (int u = 0; u < " << UNR << "; ++u) {\n";
                    b << ind << "  const " << t << " rgu = rg + u * 64;\n";
                    g.declare_coords(b, ind + "  ", rd);
                    g.decompose(b, ind + "  ", "rgu", rd);
                    for (size_t L = 0; L < expr.leaves.size(); ++L) {
                        if (g.scalar[L]) continue;
                        std::string off = g.offset(L, rd);
                        g.load_leaf(b, ind + "  ", L, "base" + std::to_string(L) + (off.empty() ? "" : " + " + off),
                                    "x" + std::to_string(L) + "[u]");
                    }
                    b << ind << "}\n";
                    b << ind << "#pragma unroll\n" << ind << "for (int u = 0; u < " << UNR << "; ++u) {\n";
                    b << ind << "#pragma unroll\n" << ind << "  for (int k = 0; k < " << V << "; ++k) {\n";
                    const std::string v = g.eval(b, ind + "    ", "u", "k");
                    if (is_sum) b << ind << "    acc[k] += " << v << ";\n";
                    else b << ind << "    ormi_am_step(mv[k], mi[k], " << v << ", (int)((rg + u * 64) * " << V << " + k));\n";
                    b << ind << "  }\n" << ind << "}\n";
                };
                b << "  " << t << " rg = rg0 + lane;\n";
                b << "  for (; rg + " << 64 * (RU - 1) << " < rg1; rg += " << 64 * RU << ") {\n";
                emit_step(RU, "    ");
                b << "  }\n";
                if (RU > 1) {
                    b << "  for (; rg < rg1; rg += 64) {\n";
                    emit_step(1, "    ");
                    b << "  }\n";
                }
                // WR > 1: the unit's waves leave their results in LDS; after the
                // barrier, lane 0 of wave q = 0 combines them in wave order.
                if (WR > 1) b << "  __shared__ float red_v_[4];\n" << (is_sum ? "" : "  __shared__ int red_i_[4];\n");
                if (is_sum) {
                    b << "  float s = " << (V > 1 ? "(acc[0] + acc[1]) + (acc[2] + acc[3])" : "acc[0]") << ";\n";
                    b << "  s = ormi_wave_sum(s);\n";
                    if (WR > 1) {
                        b << "  if (lane == 0) red_v_[wv] = s;\n  __syncthreads();\n";
                        b << "  if (!live || q != 0) return;\n";
                        b << "#pragma unroll\n  for (int w = 1; w < " << WR << "; ++w) s += red_v_[wv + w];\n";
                    }
                    b << "  if (lane == 0) {\n    ((float*)outp)[wid] = s;\n";
                    emit_epilogue(b, "    ", ep1, "s", "wid");
                    b << "  }\n";
                } else {
                    // A non-empty chain of only -inf still holds the empty marker: its first
                    // element is the first maximum. An empty chain keeps the marker, an
                    // index above every real one (R < 2^31), so it loses every tie.
                    b << "#pragma unroll\n  for (int k = 0; k < " << V << "; ++k) if (mi[k] == 0x7fffffff && rg0 + lane < rg1) mi[k] = (int)((rg0 + lane) * "
                      << V << " + k);\n";
                    b << "  float bv = mv[0]; int bi = mi[0];\n";
                    b << "#pragma unroll\n  for (int k = 1; k < " << V << "; ++k) ormi_am_take(bv, bi, mv[k], mi[k]);\n";
                    b << "  ormi_wave_argmax(bv, bi);\n";
                    if (WR > 1) {
                        b << "  if (lane == 0) { red_v_[wv] = bv; red_i_[wv] = bi; }\n  __syncthreads();\n";
                        b << "  if (!live || q != 0) return;\n";
                        b << "#pragma unroll\n  for (int w = 1; w < " << WR << "; ++w) ormi_am_take(bv, bi, red_v_[wv + w], red_i_[wv + w]);\n";
                    }
                    b << "  if (lane == 0) {\n";
                    if (is_arg) b << "    if (NP == 1) ((long long*)outp)[wid] = (long long)bi; else { ((float*)outp)[wid] = bv; outi[wid] = bi; }\n";
                    else b << "    ((float*)outp)[wid] = bv; if (NP > 1) outi[wid] = bi;\n";
                    emit_epilogue(b, "    ", ep1, "bv", "wid");
                    b << "  }\n";
                }
            }, ep1 ? ep_layout : std::string());
            if (plan.two_pass) {
                plan.workspace_bytes = (size_t)(O * P) * (sizeof(float) + sizeof(int));
                // Second pass: one wave per output row over its P partials, in part order.
                KernelLaunch& s2 = plan.second;
                Gen g2(no_expr());  // reads only the workspace
                g2.args.ptr(false, "void", "outp", out);
                g2.args.ptr(true, "float", "pvals", nullptr);
                g2.args.ptr(true, "int", "pidx", nullptr);
                declare_epilogue(g2, ep);
                g2.args.i64("NO", O);
                g2.args.i64("NP", P);
                s2.grid[0] = (uint32_t)std::max(1LL, (O + 3) / 4);
                s2.plan.kind = "row-finish";
                s2.plan.op = name;
                resolve(g2, std::string("rowfin") + name, 256, s2, [&] {
                    std::ostringstream& sb = g2.body();
                    sb << "  const int lane = threadIdx.x & 63;\n";
                    sb << "  const long long o = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);\n";
                    sb << "  if (o >= NO) return;\n";
                    sb << "  const float* pv = pvals + o * NP; const int* pi = pidx + o * NP;\n";
                    // Each lane combines its partials q = lane, lane + 64, ... in
                    // that order; sixteen are loaded before they are combined
                    // (past NP they are skipped, not added), so each batch of 1024
                    // partials costs one memory latency instead of one per load.
                    sb << "  long long q = lane;\n";
                    if (is_sum) {
                        sb << "  float s = 0.0f;\n";
                        sb << "  for (; q < NP; q += 1024) {\n    float v[16];\n#pragma unroll\n"
                              "    for (int u = 0; u < 16; ++u) v[u] = q + 64 * u < NP ? pv[q + 64 * u] : 0.0f;\n#pragma unroll\n"
                              "    for (int u = 0; u < 16; ++u) if (q + 64 * u < NP) s += v[u];\n  }\n";
                        sb << "  s = ormi_wave_sum(s);\n  if (lane == 0) {\n    ((float*)outp)[o] = s;\n";
                        emit_epilogue(sb, "    ", ep, "s", "o");
                        sb << "  }\n";
                    } else {
                        sb << "  float bv = -__builtin_inff(); int bi = 0x7fffffff;\n";
                        sb << "  for (; q < NP; q += 1024) {\n    float v[16]; int ix[16];\n#pragma unroll\n"
                              "    for (int u = 0; u < 16; ++u) { const bool in = q + 64 * u < NP; v[u] = in ? pv[q + 64 * u] : 0.0f; "
                              "ix[u] = in ? pi[q + 64 * u] : 0; }\n"
                              "#pragma unroll\n    for (int u = 0; u < 16; ++u) if (q + 64 * u < NP) ormi_am_take(bv, bi, v[u], ix[u]);\n  }\n";
                        sb << "  ormi_wave_argmax(bv, bi);\n";
                        if (is_arg) sb << "  if (lane == 0) ((long long*)outp)[o] = (long long)bi;\n";
                        else {
                            sb << "  if (lane == 0) {\n    ((float*)outp)[o] = bv;\n";
                            emit_epilogue(sb, "    ", ep, "bv", "o");
                            sb << "  }\n";
                        }
                    }
                }, ep_layout);
            }
            return plan;
        }

        // ------------------------------------------------------------ column --
        // A block is WC x WR waves: WC side by side across the kept columns
        // (each lane V consecutive columns, so a row segment is WC KB at V = 4)
        // and WR interleaved along the reduced rows. Fewer column waves when
        // the kept extent is narrow.
        const long long IG = I / V;
        int WC = 1;
        while (WC * 2 <= std::min(tn.col_cwaves, tn.col_waves) && WC * 64LL < IG) WC *= 2;
        const int WR = std::max(1, tn.col_waves / WC);
        const int W = WC * WR;
        const int block = 64 * W;
        const long long BI = (IG + 64LL * WC - 1) / (64LL * WC);
        long long P = 1;
        // Enough waves to keep HBM busy (about 16 per CU), each covering at
        // least 32 rows of its part.
        const long long target_waves = (long long)std::max(cu, 1) * 16;
        const long long waves1 = BI * O * W;
        if (waves1 < target_waves) P = std::max(1LL, std::min((target_waves + waves1 - 1) / waves1, R / (32LL * WR)));
        const long long CH = (R + P - 1) / P;
        P = R == 0 ? 1 : (R + CH - 1) / CH;
        g.choose_idx(O * I * P + R + 4LL * W * 4);
        plan.two_pass = P > 1;
        const StoreEpilogue* ep1 = plan.two_pass ? nullptr : ep;
        g.args.ptr(false, "void", "outp", plan.two_pass ? nullptr : out);
        g.args.ptr(false, "int", "outi", nullptr);
        g.declare_leaves();
        declare_epilogue(g, ep1);
        g.args.i64("NO", O);
        g.args.i64("NI", I);
        g.args.i64("NIG", IG);
        g.args.i64("NBI", BI);
        g.args.i64("NR", R);
        g.args.i64("CH", CH);
        g.declare_dims();
        g.declare_strides();
        k.grid[0] = (uint32_t)std::max(1LL, BI * O * P);
        k.plan.kind = "column";
        k.plan.op = name;
        for (auto [key, v] : {std::pair<const char*, long long>{"O", O}, {"R", R}, {"I", I}, {"vec", V}, {"waves", W},
                              {"cwaves", WC}, {"parts", P},
                              {"idx", g.idx32 ? 32 : 64}})
            k.plan.add(key, v);
        resolve(g, std::string("col") + name, block, k, [&] {
            const std::string t = g.idx();
            std::ostringstream& b = g.body();
            const int CU = tn.col_unroll;  // rows in flight per wave
            g.hoist_scalars(b, "  ");
            b << "  __shared__ float sv[" << WR << "][" << 64 * WC << "][" << V << "];\n";
            if (!is_sum) b << "  __shared__ int si[" << WR << "][" << 64 * WC << "][" << V << "];\n";
            b << "  const int lane = threadIdx.x & 63, wc = (threadIdx.x >> 6) % " << WC << ", w = (threadIdx.x >> 6) / " << WC
              << ", cl = wc * 64 + lane;\n";
            b << "  const " << t << " bid = (" << t << ")blockIdx.x;\n";
            b << "  const " << t << " bi_ = bid % (" << t << ")NBI; const " << t << " rest = bid / (" << t << ")NBI;\n";
            b << "  const " << t << " o = rest % (" << t << ")NO, p = rest / (" << t << ")NO;\n";
            b << "  const " << t << " ig = bi_ * " << 64 * WC << " + cl;\n";
            b << "  const bool active = ig < (" << t << ")NIG;\n";
            b << "  const " << t << " igc = active ? ig : (" << t << ")NIG - 1;\n";
            std::vector<int> oi = od;
            oi.insert(oi.end(), id.begin(), id.end());
            g.declare_coords(b, "  ", oi);
            g.decompose(b, "  ", "o", od);
            g.decompose(b, "  ", "igc", id);
            for (size_t L = 0; L < expr.leaves.size(); ++L) {
                if (g.scalar[L]) continue;
                std::string off = g.offset(L, oi);
                b << "  const " << t << " base" << L << " = " << (off.empty() ? "0" : off) << ";\n";
            }
            b << "  const " << t << " r0 = p * (" << t << ")CH;\n";
            b << "  const " << t << " r1 = r0 + (" << t << ")CH < (" << t << ")NR ? r0 + (" << t << ")CH : (" << t << ")NR;\n";
            if (is_sum) b << "  float acc[" << V << "];\n#pragma unroll\n  for (int k = 0; k < " << V << "; ++k) acc[k] = 0.0f;\n";
            else b << "  float bv[" << V << "]; int bx[" << V << "];\n#pragma unroll\n  for (int k = 0; k < " << V
                   << "; ++k) { bv[k] = -__builtin_inff(); bx[k] = 0x7fffffff; }\n";
            auto emit_cstep = [&](int UNR, const std::string& ind) {
                g.declare_leaf_regs(b, ind, UNR);
                b << ind << "#pragma unroll\n" << ind << "for (int u = 0; u < " << UNR << "; ++u) {\n";
                b << ind << "  const " << t << " ru = r + u * " << WR << ";\n";
                g.declare_coords(b, ind + "  ", rd);
                g.decompose(b, ind + "  ", "ru", rd);
                for (size_t L = 0; L < expr.leaves.size(); ++L) {
                    if (g.scalar[L]) continue;
                    std::string off = g.offset(L, rd);
                    g.load_leaf(b, ind + "  ", L, "base" + std::to_string(L) + (off.empty() ? "" : " + " + off), "x" + std::to_string(L) + "[u]");
                }
                b << ind << "}\n";
                b << ind << "#pragma unroll\n" << ind << "for (int u = 0; u < " << UNR << "; ++u) {\n";
                b << ind << "#pragma unroll\n" << ind << "  for (int k = 0; k < " << V << "; ++k) {\n";
                const std::string v = g.eval(b, ind + "    ", "u", "k");
                if (is_sum) b << ind << "    acc[k] += " << v << ";\n";
                else b << ind << "    ormi_am_step(bv[k], bx[k], " << v << ", (int)(r + u * " << WR << "));\n";
                b << ind << "  }\n" << ind << "}\n";
            };
            b << "  " << t << " r = r0 + w;\n";
            b << "  if (active) {\n";
            b << "    for (; r + " << WR * (CU - 1) << " < r1; r += " << WR * CU << ") {\n";
            emit_cstep(CU, "      ");
            b << "    }\n";
            b << "    for (; r < r1; r += " << WR << ") {\n";
            emit_cstep(1, "      ");
            b << "    }\n  }\n";
            if (!is_sum)  // a non-empty all -inf chain: its first element r0 + w (see the row kernel)
                b << "#pragma unroll\n  for (int k = 0; k < " << V << "; ++k) if (bx[k] == 0x7fffffff && r0 + w < r1) bx[k] = (int)(r0 + w);\n";
            b << "#pragma unroll\n  for (int k = 0; k < " << V << "; ++k) {";
            if (is_sum) b << " sv[w][cl][k] = acc[k]; }\n";
            else b << " sv[w][cl][k] = bv[k]; si[w][cl][k] = bx[k]; }\n";
            b << "  __syncthreads();\n";
            b << "  if (w == 0 && active) {\n";
            b << "    const " << t << " e0 = (p * (" << t << ")NO + o) * (" << t << ")NI + ig * " << V << ";\n";
            b << "#pragma unroll\n    for (int k = 0; k < " << V << "; ++k) {\n";
            if (is_sum) {
                b << "      float s = sv[0][cl][k];\n";
                b << "#pragma unroll\n      for (int q = 1; q < " << WR << "; ++q) s += sv[q][cl][k];\n";
                b << "      ((float*)outp)[e0 + k] = s;\n";
                emit_epilogue(b, "      ", ep1, "s", "e0 + k");
            } else {
                b << "      float v = sv[0][cl][k]; int x = si[0][cl][k];\n";
                b << "#pragma unroll\n      for (int q = 1; q < " << WR << "; ++q) ormi_am_take(v, x, sv[q][cl][k], si[q][cl][k]);\n";
                if (is_arg) b << "      if (outi == nullptr) ((long long*)outp)[e0 + k] = (long long)x; else { ((float*)outp)[e0 + k] = v; outi[e0 + k] = x; }\n";
                else b << "      ((float*)outp)[e0 + k] = v; if (outi != nullptr) outi[e0 + k] = x;\n";
                if (!is_arg) emit_epilogue(b, "      ", ep1, "v", "e0 + k");
            }
            b << "    }\n  }\n";
        }, "|cw" + std::to_string(WC) + (ep1 ? ep_layout : std::string()));
        if (plan.two_pass) {
            // Partials are laid out [P][O*I]; the second pass walks them in part order.
            plan.workspace_bytes = (size_t)(P * O * I) * (sizeof(float) + sizeof(int));
            KernelLaunch& s2 = plan.second;
            Gen g2(no_expr());  // reads only the workspace
            g2.args.ptr(false, "void", "outp", out);
            g2.args.ptr(true, "float", "pvals", nullptr);
            g2.args.ptr(true, "int", "pidx", nullptr);
            declare_epilogue(g2, ep);
            g2.args.i64("NE", O * I);
            g2.args.i64("NP", P);
            // Sums: FS lanes per column, each adding a consecutive run of parts
            // in part order, then lane 0 of the column adds the FS runs in order.
            const int FS = is_sum ? tn.col_fin_split : 1;
            s2.grid[0] = (uint32_t)std::max(1LL, (O * I * FS + 255) / 256);
            s2.plan.kind = "column-finish";
            s2.plan.op = name;
            s2.plan.add("lanes_per_column", FS);
            resolve(g2, std::string("colfin") + name + (FS > 1 ? "_s" + std::to_string(FS) : std::string()), 256, s2, [&] {
                std::ostringstream& sb = g2.body();
                // Parts are combined in part order; their loads are issued FIN at a
                // time (one round trip per FIN parts, not one per part). 16 measured
                // best: 64 loads in flight with 64-thread blocks was slower.
                constexpr int FIN = 16;
                if (FS > 1) {
                    // All lanes reach the shuffles: a lane past the last column
                    // reads column NE-1 and stores nothing.
                    sb << "  const long long ex = ((long long)blockIdx.x * 256 + threadIdx.x) / " << FS << ";\n";
                    sb << "  const int q = threadIdx.x % " << FS << ";\n";
                    sb << "  const long long e = ex < NE ? ex : NE - 1;\n";
                    sb << "  const long long run = (NP + " << FS - 1 << ") / " << FS << ", p0 = q * run;\n";
                    sb << "  const long long p1 = p0 + run < NP ? p0 + run : NP;\n";
                    sb << "  float s = 0.0f;\n  for (long long q0 = p0; q0 < p1; q0 += " << FIN << ") {\n";
                    sb << "    float v[" << FIN << "];\n";
                    sb << "#pragma unroll\n    for (int j = 0; j < " << FIN << "; ++j) v[j] = q0 + j < p1 ? pvals[(q0 + j) * NE + e] : 0.0f;\n";
                    sb << "#pragma unroll\n    for (int j = 0; j < " << FIN << "; ++j) if (q0 + j < p1) s += v[j];\n  }\n";
                    sb << "  const int lane = threadIdx.x & 63;\n";
                    sb << "  float t = s;\n";
                    sb << "#pragma unroll\n  for (int k = 1; k < " << FS << "; ++k) t += __shfl(s, lane + k, 64);\n";
                    sb << "  if (q != 0 || ex >= NE) return;\n";
                    sb << "  s = t;\n";
                    sb << "  ((float*)outp)[e] = s;\n";
                    emit_epilogue(sb, "  ", ep, "s", "e");
                    return;
                }
                sb << "  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;\n";
                sb << "  if (e >= NE) return;\n";
                if (is_sum) {
                    sb << "  float s = 0.0f;\n  for (long long q0 = 0; q0 < NP; q0 += " << FIN << ") {\n";
                    sb << "    float v[" << FIN << "];\n";
                    sb << "#pragma unroll\n    for (int j = 0; j < " << FIN << "; ++j) v[j] = q0 + j < NP ? pvals[(q0 + j) * NE + e] : 0.0f;\n";
                    sb << "#pragma unroll\n    for (int j = 0; j < " << FIN << "; ++j) if (q0 + j < NP) s += v[j];\n  }\n";
                    sb << "  ((float*)outp)[e] = s;\n";
                    emit_epilogue(sb, "  ", ep, "s", "e");
                } else {
                    sb << "  float bv = -__builtin_inff(); int bi = 0x7fffffff;\n";
                    sb << "  for (long long q0 = 0; q0 < NP; q0 += " << FIN << ") {\n";
                    sb << "    float v[" << FIN << "]; int x[" << FIN << "];\n";
                    sb << "#pragma unroll\n    for (int j = 0; j < " << FIN << "; ++j) if (q0 + j < NP) { v[j] = pvals[(q0 + j) * NE + e]; x[j] = pidx[(q0 + j) * NE + e]; }\n";
                    sb << "#pragma unroll\n    for (int j = 0; j < " << FIN << "; ++j) if (q0 + j < NP) ormi_am_take(bv, bi, v[j], x[j]);\n  }\n";
                    if (is_arg) sb << "  ((long long*)outp)[e] = (long long)bi;\n";
                    else {
                        sb << "  ((float*)outp)[e] = bv;\n";
                        emit_epilogue(sb, "  ", ep, "bv", "e");
                    }
                }
            }, ep_layout);
        }
        return plan;
    }

    // Point the split-reduction kernels at the workspace: values first, then
    // indices. The first kernel's outp/outi are args 0 and 1; the second
    // kernel's pvals/pidx are args 1 and 2.
    // ------------------------------------------------------ request cache --
    // A plan depends only on the request's structure: the tape, each leaf's
    // dtype, scalar flag and strides, the alignment of every buffer address,
    // the shape (and axes and op), the compute units and the tuning. Repeat
    // requests (every step of a training loop) take the plan from this cache and
    // rewrite only the buffer addresses (ptr_slots), skipping the generator's
    // signature and argument construction.
    namespace {
        struct KeyBuf {
            std::string s;
            KeyBuf() { s.reserve(512); }
            void i64(long long v) { s.append(reinterpret_cast<const char*>(&v), sizeof v); }
        };
        void key_expr(KeyBuf& kb, const Expr& e) {
            kb.i64((long long)e.leaves.size());
            for (const Leaf& L : e.leaves) {
                kb.i64((long long)L.dtype | ((long long)L.scalar << 8) | ((long long)L.st.size() << 16) |
                       ((long long)((uintptr_t)L.ptr & 255) << 32));
                for (long long v : L.st) kb.i64(v);
            }
            kb.i64((long long)e.insts.size());
            for (const Inst& in : e.insts)
                kb.i64((long long)in.op | ((long long)(in.a + 1) << 8) | ((long long)(in.b + 1) << 28) |
                       ((long long)in.cast << 56));
            for (int r : e.roots) kb.i64(r);
            kb.i64(-1);
        }
        struct RequestCache {
            std::mutex mu;
            std::unordered_map<std::string, KernelLaunch> maps;
            std::unordered_map<std::string, ReducePlan> reduces;
        };
        RequestCache& request_cache() {
            static auto* c = new RequestCache();
            return *c;
        }
        constexpr size_t kMaxRequests = 8192;
        // A cached launch whose kernel has been compiled since: take its handle
        // and drop the source text.
        void refresh_handle(KernelLaunch& k) {
            if (k.handle || k.key.empty()) return;
            KernelLaunch probe;
            if (cache_lookup(k.key, probe) && probe.handle) {
                k.handle = probe.handle;
                k.source.clear();
                k.source.shrink_to_fit();
            }
        }
        // The buffer address a ptr_slots source names: a leaf of the kernel's
        // expression, an output, or a store epilogue's operand.
        uint64_t slot_value(int src, const Expr& e, const void* const* outs, const Expr* ep) {
            if (src >= kEpilogueLeaf) return (uint64_t)(uintptr_t)ep->leaves[src - kEpilogueLeaf].ptr;
            return (uint64_t)(uintptr_t)(src >= 0 ? e.leaves[src].ptr : outs[-1 - src]);
        }
        // The cached launch c for this request's buffers: with launch_only and a
        // compiled kernel, only what launch() reads.
        KernelLaunch instantiate(const KernelLaunch& c, const Expr& e, const void* const* outs, bool launch_only,
                                 const Expr* ep = nullptr) {
            KernelLaunch k;
            if (!launch_only || !c.handle) {
                k = c;
            } else {
                k.handle = c.handle;
                for (int i = 0; i < 3; ++i) {
                    k.grid[i] = c.grid[i];
                    k.block[i] = c.block[i];
                }
                k.lds = c.lds;
                k.args = c.args;
            }
            for (const auto& [slot, src] : c.ptr_slots) k.args[slot] = slot_value(src, e, outs, ep);
            return k;
        }
    }  // namespace

    KernelLaunch plan_map_multi(const Expr& expr, const std::vector<int>& shape, const std::vector<void*>& outs,
                                const std::vector<DType>& out_dtypes, int cu, bool launch_only) {
        if (outs.size() != expr.roots.size() || outs.size() != out_dtypes.size() || outs.empty())
            throw std::runtime_error("HIP codegen: one output buffer and dtype per root.");
        KeyBuf kb;
        kb.i64('M');
        kb.i64(cu);
        kb.i64((long long)shape.size());
        for (int d : shape) kb.i64(d);
        for (size_t r = 0; r < outs.size(); ++r) kb.i64((long long)out_dtypes[r] | ((long long)((uintptr_t)outs[r] & 255) << 8));
        key_expr(kb, expr);
        RequestCache& rc = request_cache();
        {
            std::lock_guard<std::mutex> lock(rc.mu);
            auto it = rc.maps.find(kb.s);
            if (it != rc.maps.end()) {
                refresh_handle(it->second);
                return instantiate(it->second, expr, outs.data(), launch_only);
            }
        }
        KernelLaunch k = plan_map_multi_uncached(expr, shape, outs, out_dtypes, cu);
        std::lock_guard<std::mutex> lock(rc.mu);
        if (rc.maps.size() >= kMaxRequests) rc.maps.clear();
        rc.maps.emplace(std::move(kb.s), k);
        return k;
    }

    KernelLaunch plan_map(const Expr& expr, const std::vector<int>& shape, void* out, DType out_dtype, int cu,
                          bool launch_only) {
        return plan_map_multi(expr, shape, {out}, {out_dtype}, cu, launch_only);
    }

    ReducePlan plan_reduce(const Expr& expr, const std::vector<int>& in_shape, const std::vector<int>& axes, ReduceOp op,
                           void* out, int cu, bool launch_only, const StoreEpilogue* ep) {
        KeyBuf kb;
        kb.i64('R');
        kb.i64(cu);
        kb.i64((long long)op | ((long long)((uintptr_t)out & 255) << 8));
        kb.i64((long long)in_shape.size());
        for (int d : in_shape) kb.i64(d);
        kb.i64((long long)axes.size());
        for (int a : axes) kb.i64(a);
        key_expr(kb, expr);
        if (ep) {
            kb.i64('E');
            kb.i64((long long)ep->value | ((long long)ep->out_dtype << 32) | ((long long)((uintptr_t)ep->out & 255) << 40));
            key_expr(kb, ep->expr);
        }
        const void* outs[2] = {out, ep ? ep->out : nullptr};
        const Expr* epx = ep ? &ep->expr : nullptr;
        RequestCache& rc = request_cache();
        {
            std::lock_guard<std::mutex> lock(rc.mu);
            auto it = rc.reduces.find(kb.s);
            if (it != rc.reduces.end()) {
                refresh_handle(it->second.first);
                if (it->second.two_pass) refresh_handle(it->second.second);
                ReducePlan plan;
                plan.two_pass = it->second.two_pass;
                plan.workspace_bytes = it->second.workspace_bytes;
                plan.first = instantiate(it->second.first, expr, outs, launch_only, epx);
                if (plan.two_pass) plan.second = instantiate(it->second.second, expr, outs, launch_only, epx);
                return plan;
            }
        }
        ReducePlan plan = plan_reduce_uncached(expr, in_shape, axes, op, out, cu, ep);
        std::lock_guard<std::mutex> lock(rc.mu);
        if (rc.reduces.size() >= kMaxRequests) rc.reduces.clear();
        rc.reduces.emplace(std::move(kb.s), plan);
        return plan;
    }

    void bind_workspace(ReducePlan& plan, void* ws) {
        if (!plan.two_pass) return;
        const size_t nvals = plan.workspace_bytes / (sizeof(float) + sizeof(int));
        char* base = (char*)ws;
        const uint64_t vals = (uint64_t)(uintptr_t)base;
        const uint64_t idx = (uint64_t)(uintptr_t)(base + nvals * sizeof(float));
        plan.first.args[0] = vals;
        plan.first.args[1] = idx;
        plan.second.args[1] = vals;
        plan.second.args[2] = idx;
    }

    static std::atomic<unsigned long long> g_launches{0};
    unsigned long long kernel_launches() { return g_launches.load(); }

    void launch(const KernelLaunch& k) {
        g_launches.fetch_add(1, std::memory_order_relaxed);
        uint64_t handle = k.handle;
        if (!handle) {
            if (k.source.empty()) throw std::runtime_error("HIP codegen: kernel " + k.name + " has no source");
            std::vector<const char*> opts;
            for (const auto& o : rtc_options()) opts.push_back(o.c_str());
            ORMI_HIP_CHECK(ormi_hip_rtc_compile(k.source.c_str(), k.name.c_str(), opts.data(), (int)opts.size(), &handle));
            if (!k.key.empty()) {
                KernelLaunch done = k;
                done.handle = handle;
                cache_store(done);
            }
        }
        if (k.args.size() <= ORMI_HIP_QUEUED_MAX_ARGS) {
            ORMI_HIP_CHECK(ormi_hip_launch_queued(handle, k.grid, k.block, k.lds, k.args.data(), (int)k.args.size()));
        } else {
            std::vector<uint64_t> vals = k.args;
            std::vector<void*> ptrs(vals.size());
            for (size_t i = 0; i < vals.size(); ++i) ptrs[i] = &vals[i];
            ORMI_HIP_CHECK(ormi_hip_launch(handle, k.grid, k.block, k.lds, ptrs.data()));
        }
    }
}
