// MFMA GEMM for gfx950: C (fp32) = A . B with bf16/fp16 inputs (fp32
// accumulate) or fp32 inputs (fp32 MFMA). Replaces the reference's
// cublasSgemmBatched call (csrc/backend/cuda/kernels/blas/matmul.cu:98-105).
//
// Design
//   * Block tile BM x BN x BK, 256 threads = 4 wave64s in a 2x2 grid; each wave
//     owns a (BM/2) x (BN/2) sub-tile made of 32x32 MFMA tiles
//     (v_mfma_f32_32x32x16_{bf16,f16}, or v_mfma_f32_32x32x2_f32).
//   * Both operands sit in LDS as [mn][k] rows of BK elements plus 16 bytes of
//     padding (144-byte rows), so every MFMA operand fragment is one
//     conflict-free 16-byte ds_read per lane. Double-buffered: the next k-tile
//     is fetched from HBM into registers while the current one feeds the MFMAs.
//   * An operand whose k index is contiguous in memory ("N" for A, "T" for B)
//     is copied 16 bytes at a time. One whose m/n index is contiguous is
//     fetched as VE x VE blocks (VE = elements per 16 bytes) and transposed in
//     registers before the LDS store, so NN, NT and TN (the forward and the
//     two backward GEMMs autograd issues) all run the same MFMA loop.
//   * The tile index is remapped so the 8 XCDs (round-robin block dispatch)
//     each own a compact group of tiles, sharing operand panels in their L2.
//   * Shapes or strides the fast path cannot take (alignment, ragged 16-byte
//     chunks) run a plain tiled kernel instead.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>

#include "ormi_hip.h"
#include "ormi_hip_internal.h"

namespace ormi_hip {

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

struct GemmParams {
    const char* a;
    const char* b;
    float* c;
    int M, N, K;
    long long a_sm, a_sk, b_sk, b_sn;  // element strides
    int batch_ndim;
    int batch_shape[ORMI_GEMM_MAX_BATCH_DIMS];
    long long a_bs[ORMI_GEMM_MAX_BATCH_DIMS];
    long long b_bs[ORMI_GEMM_MAX_BATCH_DIMS];
    int tiles_m, tiles_n;
};

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

// 16-bit VE x VE transpose within one thread: out[i] holds element i of in[0..7].
__device__ __forceinline__ void transpose_8x8_b16(const u32x4_t (&in)[8], u32x4_t (&out)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const unsigned x = in[2 * e][i >> 1], y = in[2 * e + 1][i >> 1];
            out[i][e] = (i & 1) ? ((x >> 16) | (y & 0xffff0000u)) : ((x & 0xffffu) | (y << 16));
        }
    }
}
__device__ __forceinline__ void transpose_4x4_b32(const u32x4_t (&in)[4], u32x4_t (&out)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) out[i][e] = in[e][i];
}

// Registers holding one operand tile between the HBM fetch and the LDS store.
template <int NCHUNK>
struct Staged {
    u32x4_t v[NCHUNK];
};

// Fetch one BMN x BK operand tile (rows = m or n, columns = k) into registers.
// KC: k is the unit-stride index. s_mn / s_k are element strides.
template <typename Tr, int BMN, int BK, bool KC, bool EVEN>
struct TileLoader {
    static constexpr int VE = Tr::VE;
    static constexpr int KCH = BK / VE;                         // 16-byte chunks per row
    static constexpr int NCHUNK = KC ? (BMN * KCH) / 256 : VE;  // per thread
    static_assert(KC || (BMN / VE) * KCH == 256, "transposed loader needs one VE x VE block per thread");

    __device__ static void load(Staged<NCHUNK>& st, const char* base, long long s_mn, long long s_k, int mn0, int k0,
                                int MN, int K) {
        const int tid = threadIdx.x;
        if constexpr (KC) {
#pragma unroll
            for (int i = 0; i < NCHUNK; ++i) {
                const int idx = i * 256 + tid;
                const int row = idx / KCH, kc = idx % KCH;
                const int mn = mn0 + row, k = k0 + kc * VE;
                if (EVEN || (mn < MN && k < K)) {
                    st.v[i] = *(const u32x4_t*)(base + ((long long)mn * s_mn + k) * Tr::ESIZE);
                } else {
                    st.v[i] = u32x4_t{0u, 0u, 0u, 0u};
                }
            }
        } else {
            const int lane = tid & 63, wave = tid >> 6;
            const int mc = wave * 8 + (lane & 7);  // mn chunk of VE elements
            const int kb = lane >> 3;              // k block of VE rows
            const int mn = mn0 + mc * VE;
#pragma unroll
            for (int j = 0; j < VE; ++j) {
                const int k = k0 + kb * VE + j;
                if (EVEN || (mn < MN && k < K)) {
                    st.v[j] = *(const u32x4_t*)(base + ((long long)k * s_k + mn) * Tr::ESIZE);
                } else {
                    st.v[j] = u32x4_t{0u, 0u, 0u, 0u};
                }
            }
        }
    }

    // LDS tile: [BMN][KCH + 1] chunks of 16 bytes (one chunk of padding per row).
    __device__ static void store(const Staged<NCHUNK>& st, u32x4_t (*lds)[KCH + 1]) {
        const int tid = threadIdx.x;
        if constexpr (KC) {
#pragma unroll
            for (int i = 0; i < NCHUNK; ++i) {
                const int idx = i * 256 + tid;
                lds[idx / KCH][idx % KCH] = st.v[i];
            }
        } else {
            const int lane = tid & 63, wave = tid >> 6;
            const int mc = wave * 8 + (lane & 7), kb = lane >> 3;
            u32x4_t t[VE];
            if constexpr (VE == 8) transpose_8x8_b16(st.v, t);
            else transpose_4x4_b32(st.v, t);
#pragma unroll
            for (int i = 0; i < VE; ++i) lds[mc * VE + i][kb] = t[i];
        }
    }
};

template <typename Tr, int BM, int BN, int BK, bool A_KC, bool B_KC, bool EVEN>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmParams p) {
    constexpr int VE = Tr::VE, KCH = BK / VE;
    constexpr int WTM = BM / 2, WTN = BN / 2, TM = WTM / 32, TN = WTN / 32;
    using LA = TileLoader<Tr, BM, BK, A_KC, EVEN>;
    using LB = TileLoader<Tr, BN, BK, B_KC, EVEN>;

    __shared__ u32x4_t As[2][BM][KCH + 1];
    __shared__ u32x4_t Bs[2][BN][KCH + 1];

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

    // ---- batch offsets
    long long a_off = 0, b_off = 0, c_off = 0;
    {
        int bidx = blockIdx.z;
        c_off = (long long)bidx * p.M * p.N;
        for (int d = p.batch_ndim - 1; d >= 0; --d) {
            const int coord = bidx % p.batch_shape[d];
            bidx /= p.batch_shape[d];
            a_off += coord * p.a_bs[d];
            b_off += coord * p.b_bs[d];
        }
    }
    const char* a = p.a + a_off * Tr::ESIZE;
    const char* b = p.b + b_off * Tr::ESIZE;
    float* c = p.c + c_off;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int KT = (p.K + BK - 1) / BK;

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    Staged<LA::NCHUNK> sa;
    Staged<LB::NCHUNK> sb;
    LA::load(sa, a, p.a_sm, p.a_sk, m0, 0, p.M, p.K);
    LB::load(sb, b, p.b_sn, p.b_sk, n0, 0, p.N, p.K);
    LA::store(sa, As[0]);
    LB::store(sb, Bs[0]);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) {
            LA::load(sa, a, p.a_sm, p.a_sk, m0, (kt + 1) * BK, p.M, p.K);
            LB::load(sb, b, p.b_sn, p.b_sk, n0, (kt + 1) * BK, p.N, p.K);
        }
#pragma unroll
        for (int ks = 0; ks < KCH / 2; ++ks) {
            const int chunk = ks * 2 + (lane >> 5);
            u32x4_t af[TM], bfr[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = As[cur][wm * WTM + i * 32 + (lane & 31)][chunk];
#pragma unroll
            for (int j = 0; j < TN; ++j) bfr[j] = Bs[cur][wn * WTN + j * 32 + (lane & 31)][chunk];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) Tr::mma(af[i], bfr[j], acc[i][j]);
        }
        if (more) {
            LA::store(sa, As[cur ^ 1]);
            LB::store(sb, Bs[cur ^ 1]);
        }
        __syncthreads();
    }

    // ---- epilogue: 32x32 MFMA result layout, lane l / register r ->
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
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
}

// Any strides, any shape: 16x16 output tile per block, fp32 accumulation.
template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<unsigned short>(unsigned short v) { return __uint_as_float((unsigned)v << 16); }

template <typename T, bool IS_F16>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmParams p) {
    __shared__ float As[16][17];
    __shared__ float Bs[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;
    long long a_off = 0, b_off = 0;
    int bidx = blockIdx.z;
    const long long c_off = (long long)bidx * p.M * p.N;
    for (int d = p.batch_ndim - 1; d >= 0; --d) {
        const int coord = bidx % p.batch_shape[d];
        bidx /= p.batch_shape[d];
        a_off += coord * p.a_bs[d];
        b_off += coord * p.b_bs[d];
    }
    const T* a = (const T*)p.a + a_off;
    const T* b = (const T*)p.b + b_off;
    float acc = 0.0f;
    for (int k0 = 0; k0 < p.K; k0 += 16) {
        const int ar = blockIdx.y * 16 + ty, ak = k0 + tx;
        float av = 0.0f, bv = 0.0f;
        if (ar < p.M && ak < p.K) {
            const T v = a[(long long)ar * p.a_sm + (long long)ak * p.a_sk];
            if constexpr (IS_F16) { _Float16 h; __builtin_memcpy(&h, &v, 2); av = (float)h; } else av = to_f32<T>(v);
        }
        const int bk = k0 + ty, bc = blockIdx.x * 16 + tx;
        if (bk < p.K && bc < p.N) {
            const T v = b[(long long)bk * p.b_sk + (long long)bc * p.b_sn];
            if constexpr (IS_F16) { _Float16 h; __builtin_memcpy(&h, &v, 2); bv = (float)h; } else bv = to_f32<T>(v);
        }
        As[ty][tx] = av;
        Bs[ty][tx] = bv;
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) acc = __builtin_fmaf(As[ty][kk], Bs[kk][tx], acc);
        __syncthreads();
    }
    if (row < p.M && col < p.N) p.c[c_off + (long long)row * p.N + col] = acc;
}

template <typename Tr, int BM, int BN, int BK, bool A_KC, bool B_KC>
static void launch_mfma(const GemmParams& p, int batch, bool even) {
    dim3 grid(p.tiles_m * p.tiles_n, 1, batch);
    if (even) gemm_mfma_kernel<Tr, BM, BN, BK, A_KC, B_KC, true><<<grid, 256>>>(p);
    else gemm_mfma_kernel<Tr, BM, BN, BK, A_KC, B_KC, false><<<grid, 256>>>(p);
}

template <typename Tr, int BM, int BN, int BK>
static void dispatch_layout(const GemmParams& p, int batch, bool even, bool a_kc, bool b_kc) {
    if (a_kc && b_kc) launch_mfma<Tr, BM, BN, BK, true, true>(p, batch, even);
    else if (a_kc) launch_mfma<Tr, BM, BN, BK, true, false>(p, batch, even);
    else if (b_kc) launch_mfma<Tr, BM, BN, BK, false, true>(p, batch, even);
    else launch_mfma<Tr, BM, BN, BK, false, false>(p, batch, even);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace ormi_hip

using namespace ormi_hip;

extern "C" int ormi_hip_gemm(const ormi_gemm_desc* d) {
    if (!d) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: null descriptor");
    if (d->M < 0 || d->N < 0 || d->K < 0) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: negative dimension");
    if (d->batch_ndim < 0 || d->batch_ndim > ORMI_GEMM_MAX_BATCH_DIMS)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: batch_ndim must be 0..4");
    if (d->dtype != ORMI_DTYPE_F32 && d->dtype != ORMI_DTYPE_BF16 && d->dtype != ORMI_DTYPE_F16)
        return fail(ORMI_HIP_ERR_UNSUPPORTED, "ormi_hip_gemm: dtype must be f32, bf16 or f16");
    long long batch = 1;
    for (int i = 0; i < d->batch_ndim; ++i) {
        if (d->batch_shape[i] <= 0) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: batch extents must be positive");
        batch *= d->batch_shape[i];
    }
    if (batch > 65535) return fail(ORMI_HIP_ERR_UNSUPPORTED, "ormi_hip_gemm: more than 65535 batches");
    if ((long long)d->M * d->N == 0) return ORMI_HIP_OK;
    if (!d->a || !d->b || !d->c) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: null operand");
    int rc = ensure_init();
    if (rc != ORMI_HIP_OK) return rc;

    GemmParams p{};
    p.a = (const char*)d->a;
    p.b = (const char*)d->b;
    p.c = d->c;
    p.M = d->M; p.N = d->N; p.K = d->K;
    p.a_sm = d->a_stride_m; p.a_sk = d->a_stride_k;
    p.b_sk = d->b_stride_k; p.b_sn = d->b_stride_n;
    p.batch_ndim = d->batch_ndim;
    for (int i = 0; i < d->batch_ndim; ++i) {
        p.batch_shape[i] = d->batch_shape[i];
        p.a_bs[i] = d->a_batch_stride[i];
        p.b_bs[i] = d->b_batch_stride[i];
    }

    if (d->K == 0) {
        const float zero = 0.0f;
        return ormi_hip_fill(d->c, &zero, 4, (size_t)batch * d->M * d->N);
    }

    const bool f32 = d->dtype == ORMI_DTYPE_F32;
    const int VE = f32 ? 4 : 8;
    // Which index is unit-stride for each operand (k preferred when both are).
    const bool a_kc = d->a_stride_k == 1, a_mc = d->a_stride_m == 1 || d->M == 1;
    const bool b_kc = d->b_stride_k == 1, b_nc = d->b_stride_n == 1 || d->N == 1;
    bool fast = (a_kc || a_mc) && (b_kc || b_nc) && aligned16(d->a) && aligned16(d->b);
    if (fast) {
        // 16-byte chunks must be whole: the unit-stride extent and every other
        // stride a multiple of VE elements.
        const long long a_other = a_kc ? d->a_stride_m : d->a_stride_k;
        const long long b_other = b_kc ? d->b_stride_n : d->b_stride_k;
        const int a_unit_extent = a_kc ? d->K : d->M;
        const int b_unit_extent = b_kc ? d->K : d->N;
        fast = (a_other % VE == 0) && (b_other % VE == 0) && (a_unit_extent % VE == 0) && (b_unit_extent % VE == 0);
        for (int i = 0; i < d->batch_ndim && fast; ++i)
            fast = (d->a_batch_stride[i] % VE == 0) && (d->b_batch_stride[i] % VE == 0);
    }

    if (!fast) {
        dim3 grid((d->N + 15) / 16, (d->M + 15) / 16, (unsigned)batch);
        if (f32) gemm_generic_kernel<float, false><<<grid, 256>>>(p);
        else if (d->dtype == ORMI_DTYPE_BF16) gemm_generic_kernel<unsigned short, false><<<grid, 256>>>(p);
        else gemm_generic_kernel<unsigned short, true><<<grid, 256>>>(p);
    } else if (f32) {
        constexpr int BM = 128, BN = 128, BK = 32;
        p.tiles_m = (d->M + BM - 1) / BM;
        p.tiles_n = (d->N + BN - 1) / BN;
        const bool even = d->M % BM == 0 && d->N % BN == 0 && d->K % BK == 0;
        dispatch_layout<TrF32, BM, BN, BK>(p, (int)batch, even, a_kc, b_kc);
    } else {
        constexpr int BM = 256, BN = 256, BK = 64;
        p.tiles_m = (d->M + BM - 1) / BM;
        p.tiles_n = (d->N + BN - 1) / BN;
        const bool even = d->M % BM == 0 && d->N % BN == 0 && d->K % BK == 0;
        if (d->dtype == ORMI_DTYPE_BF16) dispatch_layout<TrBF16, BM, BN, BK>(p, (int)batch, even, a_kc, b_kc);
        else dispatch_layout<TrF16, BM, BN, BK>(p, (int)batch, even, a_kc, b_kc);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("ormi_hip_gemm launch: ") + hipGetErrorString(e));
    return ORMI_HIP_OK;
}
