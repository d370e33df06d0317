// Shared by gemm.hip and gemm_epi.hip: GEMM parameters, the element-wise
// epilogue, the register-staged MFMA kernel (gemm_mfma_kernel) and its tile
// loader. Each translation unit instantiates a disjoint set of kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

#include "ormi_hip.h"
#include "device/ormi_device.h"

namespace ormi_hip {

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) char lds_char;

// Wait until at most V vector-memory instructions of this wave are pending.
template <int V>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(V >= 0 && V < 64, "vmcnt is a 6-bit counter");
    // s_waitcnt encoding: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] at [15:14];
    // expcnt and lgkmcnt at their maxima (no wait).
    __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | (7 << 4) | (15 << 8));
}
// The same with lgkmcnt(0): this wave's LDS reads have also completed.
template <int V>
__device__ __forceinline__ void wait_vmcnt_lds() {
    static_assert(V >= 0 && V < 64, "vmcnt is a 6-bit counter");
    __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | (7 << 4));
}
// Workgroup barrier that orders LDS accesses in program order for the
// compiler without waiting for outstanding vector-memory loads (a C++
// __syncthreads() would also drain the direct loads of later stages).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Element-wise epilogue (ormi_hip_gemm_ex). kind is ORMI_GEMM_EPI_NONE in the
// GEMM kernels whenever the epilogue runs in gemm_finish_kernel instead.
struct Epi {
    int kind, fn, form;
    const float* s;
    const float* d;
    long long d_sm, d_sn;
    long long d_bs[ORMI_GEMM_MAX_BATCH_DIMS];
    float* aux;
};

struct GemmParams {
    const char* a;
    const char* b;
    float* c;          // final output, or the split-K workspace
    int M, N, K;
    long long a_sm, a_sk, b_sk, b_sn;  // element strides
    int batch_ndim;
    int batch_shape[ORMI_GEMM_MAX_BATCH_DIMS];
    long long a_bs[ORMI_GEMM_MAX_BATCH_DIMS];
    long long b_bs[ORMI_GEMM_MAX_BATCH_DIMS];
    int tiles_m, tiles_n;
    int batch;         // number of batches
    int splits;        // K splits (1 = write C directly)
    int k_per_split;   // multiple of BK
    Epi epi;
};

// The ORMI_GEMM_FN_* functions: the device helpers the fused element-wise
// kernels call for the same ops, so a fused epilogue rounds identically.
__device__ __forceinline__ float epi_fn(int fn, float x) {
    switch (fn) {
        case ORMI_GEMM_FN_RELU: return ormi_relu(x);
        case ORMI_GEMM_FN_STEP: return ormi_step(x);
        case ORMI_GEMM_FN_TANH: return ormi_tanh(x);
        case ORMI_GEMM_FN_TANH_GRAD: return ormi_tanh_grad(x);
        case ORMI_GEMM_FN_SIGMOID: return ormi_sigmoid(x);
        case ORMI_GEMM_FN_SIGMOID_GRAD: return ormi_sigmoid_grad(x);
        case ORMI_GEMM_FN_GELU: return ormi_gelu(x);
        case ORMI_GEMM_FN_GELU_GRAD: return ormi_gelu_grad(x);
        default: return x;
    }
}

// epi_fn with the function fixed at compile time.
template <int FN>
__device__ __forceinline__ float epi_fn_t(float x) {
    if constexpr (FN == ORMI_GEMM_FN_RELU) return ormi_relu(x);
    else if constexpr (FN == ORMI_GEMM_FN_STEP) return ormi_step(x);
    else if constexpr (FN == ORMI_GEMM_FN_TANH) return ormi_tanh(x);
    else if constexpr (FN == ORMI_GEMM_FN_TANH_GRAD) return ormi_tanh_grad(x);
    else if constexpr (FN == ORMI_GEMM_FN_SIGMOID) return ormi_sigmoid(x);
    else if constexpr (FN == ORMI_GEMM_FN_SIGMOID_GRAD) return ormi_sigmoid_grad(x);
    else if constexpr (FN == ORMI_GEMM_FN_GELU) return ormi_gelu(x);
    else if constexpr (FN == ORMI_GEMM_FN_GELU_GRAD) return ormi_gelu_grad(x);
    else return x;
}

template <int V>
struct FnConst {
    static constexpr int value = V;
};

// The functions the in-store epilogue is instantiated for (the ones the HIP
// scheduler fuses); epi_in_store says whether an epilogue is among them.
template <class G>
__device__ __forceinline__ void epi_dispatch_unary(int fn, G&& g) {
    switch (fn) {
        case ORMI_GEMM_FN_RELU: g(FnConst<ORMI_GEMM_FN_RELU>{}); break;
        case ORMI_GEMM_FN_TANH: g(FnConst<ORMI_GEMM_FN_TANH>{}); break;
        case ORMI_GEMM_FN_SIGMOID: g(FnConst<ORMI_GEMM_FN_SIGMOID>{}); break;
        default: g(FnConst<ORMI_GEMM_FN_GELU>{}); break;
    }
}
template <class G>
__device__ __forceinline__ void epi_dispatch_grad(int fn, G&& g) {
    switch (fn) {
        case ORMI_GEMM_FN_STEP: g(FnConst<ORMI_GEMM_FN_STEP>{}); break;
        case ORMI_GEMM_FN_TANH_GRAD: g(FnConst<ORMI_GEMM_FN_TANH_GRAD>{}); break;
        case ORMI_GEMM_FN_SIGMOID_GRAD: g(FnConst<ORMI_GEMM_FN_SIGMOID_GRAD>{}); break;
        case ORMI_GEMM_FN_GELU_GRAD: g(FnConst<ORMI_GEMM_FN_GELU_GRAD>{}); break;
        default: g(FnConst<ORMI_GEMM_FN_IDENTITY>{}); break;
    }
}
inline bool epi_in_store(const Epi& e) {
    if (e.kind == ORMI_GEMM_EPI_UNARY)
        return e.fn == ORMI_GEMM_FN_RELU || e.fn == ORMI_GEMM_FN_TANH || e.fn == ORMI_GEMM_FN_SIGMOID || e.fn == ORMI_GEMM_FN_GELU;
    if (e.kind == ORMI_GEMM_EPI_MUL_FN_D)
        return e.fn == ORMI_GEMM_FN_IDENTITY || e.fn == ORMI_GEMM_FN_STEP || e.fn == ORMI_GEMM_FN_TANH_GRAD ||
               e.fn == ORMI_GEMM_FN_SIGMOID_GRAD || e.fn == ORMI_GEMM_FN_GELU_GRAD;
    return e.kind == ORMI_GEMM_EPI_ADD;
}

__host__ __device__ __forceinline__ bool epi_reads_d(const Epi& e) {
    return e.kind == ORMI_GEMM_EPI_ADD || e.kind == ORMI_GEMM_EPI_MUL_FN_D;
}

// Store product v of one output element: C[ci] (and aux[ci]) in C's layout;
// dv is that element's D value (read beforehand when epi_reads_d), sv the
// scale s[0] when the epilogue has one. Every HIP translation unit is
// compiled with -ffp-contract=off, so each operation below rounds on its own,
// as in the unfused element-wise kernel.
__device__ __forceinline__ void epi_store(const Epi& e, float sv, float* c, float* aux, long long ci, float dv, float v) {
    switch (e.kind) {
        case ORMI_GEMM_EPI_ADD: {
            const float t = e.s ? v * sv : v;
            c[ci] = e.form == 0 ? dv + t : e.form == 1 ? dv - t : t - dv;
            break;
        }
        case ORMI_GEMM_EPI_UNARY:
            if (aux) aux[ci] = v;
            c[ci] = epi_fn(e.fn, v);
            break;
        case ORMI_GEMM_EPI_MUL_FN_D:
            c[ci] = v * epi_fn(e.fn, dv);
            break;
        default:
            c[ci] = v;
    }
}

// Element-type traits: storage size, elements per 16 bytes, MFMA step.
struct TrBF16 {
    static constexpr int ESIZE = 2, VE = 8;
    __device__ static void mma(const u32x4_t& a, const u32x4_t& b, f32x16_t& acc) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
    }
};
struct TrF16 {
    static constexpr int ESIZE = 2, VE = 8;
    __device__ static void mma(const u32x4_t& a, const u32x4_t& b, f32x16_t& acc) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), acc, 0, 0, 0);
    }
};
struct TrF32 {
    static constexpr int ESIZE = 4, VE = 4;
    // One 16-byte fragment holds 4 consecutive k per lane: four K=2 MFMAs.
    // Lane half h and step s cover k = 4h + s of the 8-k group, identically
    // for A and B, so every k is paired with itself.
    __device__ static void mma(const u32x4_t& a, const u32x4_t& b, f32x16_t& acc) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[s]), __uint_as_float(b[s]), acc, 0, 0, 0);
    }
};

// Fetch one BMN x BK operand tile (rows = m or n, columns = k) into registers
// and store it to LDS. KC: k is the unit-stride index. NT: threads per block.
// LDS layouts, both giving each lane a 16-byte MFMA fragment of 4 consecutive
// k (chunk ch holds k = 4 ch .. 4 ch + 3) of one m / n row:
//   KC, and 16-bit mn-contiguous: [BMN][KCH + 1] 16-byte chunks; 16-bit
//       mn-contiguous tiles are transposed in registers on the way.
//   32-bit mn-contiguous (KMN): [BK][BMN + 8] floats, stored as loaded (each
//       k-row is one contiguous run, so the stores cannot conflict); a
//       fragment is 4 dword reads. The lane halves of a read sit 4 k-rows =
//       4 (BMN + 8) dwords apart, an odd multiple of 32 banks of the 64, so
//       they do not conflict either.
template <typename Tr, int BMN, int BK, bool KC, bool EVEN, int NT>
struct TileLoader {
    static constexpr int VE = Tr::VE, ES = Tr::ESIZE;
    static constexpr int KCH = BK / VE;  // 16-byte chunks per row
    static constexpr bool KMN = !KC && ES == 4;
    static constexpr int PITCH = BMN + 8;  // KMN row pitch in floats
    static_assert(!KMN || (4 * PITCH) % 64 == 32, "KMN pitch must put lane halves 32 banks apart");
    static constexpr int LDS_BYTES = KMN ? BK * PITCH * 4 : BMN * (KCH + 1) * 16;
    // Direct copy: 16-byte chunks per thread.
    static constexpr int NCHUNK = (BMN * KCH) / NT;
    // Transposed copy: each thread owns VE k-rows x MC mn-elements.
    static constexpr int MC = (BMN * BK) / (VE * NT);
    static constexpr int MCW = MC * ES / 4;  // dwords per k-row
    static constexpr int MCU = BMN / (MC > 0 ? MC : 1);  // mn units per k-row (KMN)
    static constexpr int NREG = KC ? NCHUNK * 4 : VE * MCW;
    static_assert(KC ? (NCHUNK >= 1 && NCHUNK * NT == BMN * KCH) : (KCH == 8 && MC >= 1 && MC * VE * NT == BMN * BK && MCW >= 1),
                  "tile / thread-count combination not supported");
    static_assert(!KMN || (MCU % 32 == 0 && MCU * MC == BMN), "KMN needs whole half-waves per k-row");
    // load() moves 4, 2 or 1 dwords per k-row of an mn-contiguous tile.
    static_assert(KC || MCW == 4 || MCW == 2 || MCW == 1, "mn-contiguous tiles need 1, 2 or 4 dwords per thread and k-row");

    unsigned r[NREG];

    // Thread -> (mn unit of MC elements, k block of VE rows) for mn-contiguous tiles.
    __device__ static int unit_mn() {
        const int tid = threadIdx.x;
        if constexpr (KMN) return tid % MCU;
        else return (tid >> 6) * 8 + (tid & 7);
    }
    __device__ static int unit_kb() {
        const int tid = threadIdx.x;
        if constexpr (KMN) return tid / MCU;
        else return (tid & 63) >> 3;
    }

    // The 16-byte fragment of mn-row `row`, chunk `ch`.
    __device__ static u32x4_t frag(const char* lds, int row, int ch) {
        if constexpr (KMN) {
            const unsigned* f = (const unsigned*)lds + ch * 4 * PITCH + row;
            return u32x4_t{f[0], f[PITCH], f[2 * PITCH], f[3 * PITCH]};
        } else {
            return ((const u32x4_t*)lds)[row * (KCH + 1) + ch];
        }
    }

    __device__ void load(const char* base, long long s_mn, long long s_k, int mn0, int k0, int MN, int K) {
        const int tid = threadIdx.x;
        if constexpr (KC) {
#pragma unroll
            for (int i = 0; i < NCHUNK; ++i) {
                const int idx = i * NT + tid;
                const int row = idx / KCH, kc = idx % KCH;
                const int mn = mn0 + row, k = k0 + kc * VE;
                u32x4_t v = {0u, 0u, 0u, 0u};
                if (EVEN || (mn < MN && k < K)) v = *(const u32x4_t*)(base + ((long long)mn * s_mn + k) * ES);
#pragma unroll
                for (int e = 0; e < 4; ++e) r[i * 4 + e] = v[e];
            }
        } else {
            const int mc = unit_mn(), kb = unit_kb();
            const int mn = mn0 + mc * MC;
#pragma unroll
            for (int j = 0; j < VE; ++j) {
                const int k = k0 + kb * VE + j;
                const bool ok = EVEN || (mn < MN && k < K);
                const char* p = base + ((long long)k * s_k + mn) * ES;
                if constexpr (MCW == 4) {
                    u32x4_t v = {0u, 0u, 0u, 0u};
                    if (ok) v = *(const u32x4_t*)p;
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[j * 4 + e] = v[e];
                } else if constexpr (MCW == 2) {
                    typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
                    u32x2_t v = {0u, 0u};
                    if (ok) v = *(const u32x2_t*)p;
                    r[j * 2] = v[0];
                    r[j * 2 + 1] = v[1];
                } else {
                    r[j] = ok ? *(const unsigned*)p : 0u;
                }
            }
        }
    }

    __device__ void store(char* smem) const {
        const int tid = threadIdx.x;
        if constexpr (KC) {
            u32x4_t (*lds)[KCH + 1] = (u32x4_t (*)[KCH + 1])smem;
#pragma unroll
            for (int i = 0; i < NCHUNK; ++i) {
                const int idx = i * NT + tid;
                lds[idx / KCH][idx % KCH] = u32x4_t{r[i * 4], r[i * 4 + 1], r[i * 4 + 2], r[i * 4 + 3]};
            }
        } else if constexpr (KMN) {
            const int mc = unit_mn(), kb = unit_kb();
            unsigned* row0 = (unsigned*)smem + (kb * VE) * PITCH + mc * MC;
#pragma unroll
            for (int j = 0; j < VE; ++j) {
                unsigned* d = row0 + j * PITCH;
                if constexpr (MCW == 4) {
                    *(u32x4_t*)d = u32x4_t{r[j * 4], r[j * 4 + 1], r[j * 4 + 2], r[j * 4 + 3]};
                } else if constexpr (MCW == 2) {
                    typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
                    *(u32x2_t*)d = u32x2_t{r[j * 2], r[j * 2 + 1]};
                } else {
                    *d = r[j];
                }
            }
        } else {
            // 16-bit mn-contiguous: element i of k-row j is half (i & 1) of
            // dword i / 2 of that row.
            static_assert(ES == 2, "32-bit mn-contiguous tiles use the KMN layout");
            u32x4_t (*lds)[KCH + 1] = (u32x4_t (*)[KCH + 1])smem;
            const int mc = unit_mn(), kb = unit_kb();
#pragma unroll
            for (int i = 0; i < MC; ++i) {
                u32x4_t t;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const unsigned x = r[(2 * e) * MCW + (i >> 1)], y = r[(2 * e + 1) * MCW + (i >> 1)];
                    t[e] = (i & 1) ? ((x >> 16) | (y & 0xffff0000u)) : ((x & 0xffffu) | (y << 16));
                }
                lds[mc * MC + i][kb] = t;
            }
        }
    }
};

// EPI: the store applies p.epi (only instantiated for the configurations the
// fp32 dispatch picks by default; the others leave epilogues to the finish pass).
// Epilogue of one wave's TM x TN 32x32 accumulator blocks, all in bounds:
// block (i, j) covers rows row0 + 32 i .. and columns col0 + 32 j .. of C
// (row stride ldc); lane l / register r holds row 8*(r/4) + 4*(l/32) + r%4,
// column l%32. dd points at D's element (0, 0) for this batch (strides e.d_sm,
// e.d_sn); aux, when set, shares C's layout. D values are loaded ahead of the
// stores that need them: loads and stores retire through one in-order
// counter, so a load issued after a store would wait out a memory latency per
// element. EARLY_D: dv already holds them (loaded during the last k-tile);
// otherwise 32x32 block t + 1's are loaded before block t is stored (a lane's
// blocks are distinct elements, so this holds when D is C itself).
// ONLY >= 0 compiles in that epilogue kind alone (the caller guarantees e.kind).
template <int TM, int TN, bool EARLY_D, int ONLY = -1>
__device__ __forceinline__ void epi_tile(const Epi& e, float sv, float* c, float* aux, const float* dd, int ldc, int row0,
                                         int col0, const f32x16_t (&acc)[TM][TN], float (&dv)[TM][TN][16], bool reads_d) {
    const int lane = threadIdx.x & 63;
    if (!reads_d) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) dv[i][j][r] = 0.0f;
    }
    auto load_sub = [&](float (&dst)[16], int i, int j) {
        const int col = col0 + j * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = row0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            dst[r] = dd[row * e.d_sm + col * e.d_sn];
        }
    };
    // One unrolled store loop per (kind, function, aux), chosen once:
    // a run-time dispatch inside the loop costs more than the arithmetic.
    auto each = [&](auto&& op) {
        float dn[16];
        if (!EARLY_D && reads_d) load_sub(dn, 0, 0);
#pragma unroll
        for (int t = 0; t < TM * TN; ++t) {
            const int i = t / TN, j = t % TN;
            float dc[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) dc[r] = (EARLY_D || !reads_d) ? dv[i][j][r] : dn[r];
            if (!EARLY_D && reads_d && t + 1 < TM * TN) load_sub(dn, (t + 1) / TN, (t + 1) % TN);
            const int col = col0 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = row0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                op((long long)row * ldc + col, dc[r], acc[i][j][r]);
            }
        }
    };
    const int kind = ONLY >= 0 ? ONLY : e.kind;
    if constexpr (ONLY < 0 || ONLY == ORMI_GEMM_EPI_ADD) {
        if (kind == ORMI_GEMM_EPI_ADD) {
            const bool scaled = e.s != nullptr;
            const int form = e.form;
            each([&](long long ci, float d, float v) {
                const float t = scaled ? v * sv : v;
                c[ci] = form == 0 ? d + t : form == 1 ? d - t : t - d;
            });
            return;
        }
    }
    if constexpr (ONLY < 0 || ONLY == ORMI_GEMM_EPI_UNARY) {
        if (kind == ORMI_GEMM_EPI_UNARY) {
            epi_dispatch_unary(e.fn, [&](auto fn) {
                if (aux) each([&](long long ci, float, float v) { aux[ci] = v; c[ci] = epi_fn_t<decltype(fn)::value>(v); });
                else each([&](long long ci, float, float v) { c[ci] = epi_fn_t<decltype(fn)::value>(v); });
            });
            return;
        }
    }
    if constexpr (ONLY < 0 || ONLY == ORMI_GEMM_EPI_MUL_FN_D) {
        epi_dispatch_grad(e.fn, [&](auto fn) {
            each([&](long long ci, float d, float v) { c[ci] = v * epi_fn_t<decltype(fn)::value>(d); });
        });
    }
}

template <typename Tr, int BM, int BN, int BK, int WGM, int WGN, bool A_KC, bool B_KC, bool EVEN, bool EPI = false>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_mfma_kernel(GemmParams p) {
    constexpr int NT = 64 * WGM * WGN;
    constexpr int VE = Tr::VE, KCH = BK / VE;
    constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
    static_assert(TM >= 1 && TN >= 1 && KCH % 2 == 0, "bad tile shape");
    static_assert(!EPI || EVEN, "epilogue kernels read D unguarded: whole tiles only");
    using LA = TileLoader<Tr, BM, BK, A_KC, EVEN, NT>;
    using LB = TileLoader<Tr, BN, BK, B_KC, EVEN, NT>;

    __shared__ __attribute__((aligned(16))) char As[2][LA::LDS_BYTES];
    __shared__ __attribute__((aligned(16))) char Bs[2][LB::LDS_BYTES];

    // ---- tile index: XCD-aware remap, then groups of 4 tile rows.
    const int T = p.tiles_m * p.tiles_n;
    int t = blockIdx.x;
    if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
    constexpr int GROUP = 4;
    const int group_size = GROUP * p.tiles_n;
    const int g = t / group_size, first_m = g * GROUP;
    const int gm = min(p.tiles_m - first_m, GROUP);
    const int tm_idx = first_m + (t % group_size) % gm;
    const int tn_idx = (t % group_size) / gm;
    const int m0 = tm_idx * BM, n0 = tn_idx * BN;

    // ---- batch and K split
    const int split = blockIdx.z % p.splits;
    int bidx = blockIdx.z / p.splits;
    long long a_off = 0, b_off = 0, d_off = 0;
    const long long c_off = ((long long)split * p.batch + bidx) * p.M * p.N;
    for (int d = p.batch_ndim - 1; d >= 0; --d) {
        const int coord = bidx % p.batch_shape[d];
        bidx /= p.batch_shape[d];
        a_off += coord * p.a_bs[d];
        b_off += coord * p.b_bs[d];
        d_off += coord * p.epi.d_bs[d];
    }
    const char* a = p.a + a_off * Tr::ESIZE;
    const char* b = p.b + b_off * Tr::ESIZE;
    float* c = p.c + c_off;
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int KT = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    LA la;
    LB lb;
    if (KT > 0) {
        la.load(a, p.a_sm, p.a_sk, m0, kbeg, p.M, kend);
        lb.load(b, p.b_sn, p.b_sk, n0, kbeg, p.N, kend);
        la.store(As[0]);
        lb.store(Bs[0]);
    }
    __syncthreads();

    // Epilogue operand D (EPI kernels run only for shapes in whole tiles, so
    // every element is in bounds). With at most 32 values per lane it is read
    // during the last k-tile: its latency, and the D-only part of the
    // epilogue, overlap the last MFMAs instead of adding to the tail every CU
    // reaches at once. 64 values kept live through the loop would spill.
    float dv[EPI ? TM : 1][EPI ? TN : 1][16];
    const bool reads_d = EPI && epi_reads_d(p.epi);
    constexpr bool EARLY_D = TM * TN <= 2;

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) {
            la.load(a, p.a_sm, p.a_sk, m0, kbeg + (kt + 1) * BK, p.M, kend);
            lb.load(b, p.b_sn, p.b_sk, n0, kbeg + (kt + 1) * BK, p.N, kend);
        }
        if constexpr (EPI && EARLY_D) {
            if (!more && reads_d) {
                const float* dd = p.epi.d + d_off;
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        const int col = n0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                            dv[i][j][r] = dd[row * p.epi.d_sm + col * p.epi.d_sn];
                        }
                    }
            }
        }
        u32x4_t af[2][TM], bfr[2][TN];
        const int half = lane >> 5, row = lane & 31;
#pragma unroll
        for (int i = 0; i < TM; ++i) af[0][i] = LA::frag(As[cur], wm * WTM + i * 32 + row, half);
#pragma unroll
        for (int j = 0; j < TN; ++j) bfr[0][j] = LB::frag(Bs[cur], wn * WTN + j * 32 + row, half);
#pragma unroll
        for (int ks = 0; ks < KCH / 2; ++ks) {
            const int q = ks & 1;
            if (ks + 1 < KCH / 2) {
                const int chunk = (ks + 1) * 2 + half;
#pragma unroll
                for (int i = 0; i < TM; ++i) af[q ^ 1][i] = LA::frag(As[cur], wm * WTM + i * 32 + row, chunk);
#pragma unroll
                for (int j = 0; j < TN; ++j) bfr[q ^ 1][j] = LB::frag(Bs[cur], wn * WTN + j * 32 + row, chunk);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) Tr::mma(af[q][i], bfr[q][j], acc[i][j]);
            // The next tile goes to the other LDS buffer halfway through this
            // tile's MFMAs: every wave finished reading that buffer before the
            // previous barrier, and its write latency now overlaps matrix work.
            if (ks == KCH / 4 - 1 && more) {
                la.store(As[cur ^ 1]);
                lb.store(Bs[cur ^ 1]);
            }
        }
        // After the last tile nothing touches LDS again.
        if (more) __syncthreads();
    }

    // ---- epilogue: 32x32 MFMA result layout, lane l / register r ->
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
    if constexpr (!EPI) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = n0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (EVEN || (row < p.M && col < p.N)) c[(long long)row * p.N + col] = acc[i][j][r];
                }
            }
        }
    } else {
        // Only without a K split (the host runs the finish pass otherwise),
        // so c_off is the batch offset and aux shares it.
        epi_tile<TM, TN, EARLY_D>(p.epi, p.epi.s ? *p.epi.s : 0.0f, c, p.epi.aux ? p.epi.aux + c_off : nullptr, p.epi.d + d_off, p.N,
                                  m0 + wm * WTM, n0 + wn * WTN, acc, dv, reads_d);
    }
}

// Launch gemm_mfma_kernel with the epilogue in its store: fp32 configuration
// 2 or 3, M, N and K in whole tiles (gemm_epi.hip).
void run32_epi(int id, const GemmParams& p, dim3 grid, bool a_kc, bool b_kc);
// fp32 GEMM with direct HBM->LDS loads (gemm_f32dma.hip): tile extents and
// depth of configuration id, and its launch. K must be a multiple of the
// depth, and an mn-contiguous operand's extent a multiple of 4.
void cfg32_dma(int id, int* bm, int* bn, int* bk);
// epi: apply p.epi in the store (M, N and K in whole tiles, no K split).
void run32_dma(int id, const GemmParams& p, dim3 grid, bool a_kc, bool b_kc, bool epi);
// The persistent form of the default direct-load configuration (1): `groups`
// work-groups walk the p.tiles_m x p.tiles_n tiles; whole tiles, one batch,
// no K split; p.epi (its kind compiled in) applied in the store.
void run32_dma_persist(const GemmParams& p, int groups, bool a_kc, bool b_kc);
// Two independent products of configuration 1 as one persistent launch of
// `groups` work-groups (each in whole tiles, one batch, no K split, the
// epilogue in the store); false, with nothing launched, when the pair of
// layouts and epilogue kinds is not one the kernel is instantiated for.
bool run32_dma_pair(const GemmParams& p0, bool a_kc0, bool b_kc0, const GemmParams& p1, bool a_kc1, bool b_kc1,
                    int groups);

}  // namespace ormi_hip
