// MFMA GEMM for gfx950: C (fp32) = A . B with bf16/fp16 inputs (fp32
// accumulate) or fp32 inputs (fp32 MFMA). Replaces the reference's
// cublasSgemmBatched call (csrc/backend/cuda/kernels/blas/matmul.cu:98-105).
//
// Kernels, in the order the dispatch (gemm_run_locked) prefers them
//   * 16-bit direct-load kernels (this file): HBM -> LDS with
//     global_load_lds_dwordx4 into XOR-swizzled multi-stage rings, 4 waves of
//     128x128 (256x256 tiles) or 64x64 (128x128 tiles), 32x32x16 MFMAs. A
//     k-contiguous A with K a multiple of 64 takes whole 128-byte lines per
//     row (gemm_ilp_kernel, 64-deep A slots); otherwise the interleaved kernel
//     (gemm_il_kernel). 256x256 tiles when there are at least as many as
//     compute units, else 128x128.
//   * fp32 direct-load kernels (gemm_f32dma.hip): 8 waves of 64x32 on
//     128x128x32 tiles and 32x32x2 fp32 MFMAs; a persistent form walks several
//     tiles per work-group through one ring when the output has more tiles
//     than compute units.
//   * Operands those kernels cannot take as given (a unit-stride extent or
//     another stride not in whole 16-byte chunks, no unit stride, K not in
//     whole tiles) are packed into zero-padded k-contiguous buffers first for
//     large products (gemm_packed_locked).
//   * Register-staged kernels (gemm_mfma_kernel, gemm_mfma.h) and a plain tiled
//     kernel cover what remains (small products, the allocation-free entry's
//     unpackable layouts).
// Shared by all
//   * An element-wise epilogue (ormi_hip_gemm_ex) is applied in the store of
//     the fp32 direct-load kernels (gemm_f32dma.hip, gemm_epi.hip), otherwise
//     in the pass that finishes a K split.
//   * The tile index is remapped so the 8 XCDs (round-robin block dispatch)
//     each own a compact group of tiles, sharing operand panels in their L2.
//   * When the output has too few tiles to occupy the 256 CUs, K is split
//     across blocks; partial products go to a workspace and a second kernel
//     adds them in split order (deterministic).
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <string>

#include "ormi_hip.h"
#include "ormi_hip_internal.h"
#include "gemm_mfma.h"

namespace ormi_hip {

// ------------------------------------------------------------------------
// 16-bit GEMM with direct HBM->LDS loads (gfx950 global_load_lds_dwordx4).
//
// Each load instruction moves 64 lanes x 16 bytes into 1 KB of LDS in lane
// order, so tiles are stored unpadded and bank conflicts are avoided with XOR
// swizzles of the 16-byte chunk index instead (BK = tile depth, 32 or 64):
//   k-contiguous operand  [BMN][BK]  2*BK-byte rows, physical chunk = c ^ swz_k(row),
//       BK 64: swz_k(r) = (r & 7) ^ ((r >> 3) & 1);
//       BK 32: swz_k(r) = ((r >> 1) & 3) ^ ((r >> 3) & 1);
//       16 consecutive rows read by one ds_read_b128 land on distinct banks
//       for 32- and 64-bank LDS;
//   mn-contiguous operand [BK][BMN]  BMN*2-byte rows, physical chunk = c ^ swz_mn(k),
//       swz_mn(k) = 4 * (k & 3): the 4 rows x 4 chunks one transpose read
//       touches cover 64 distinct banks.
// The mn-contiguous operand is read with ds_read_b64_tr_b16: in each 16-lane
// group, output lane j slot s is input lane (4s + j/4) element (j % 4); with
// input lane i pointing at [kbase + i/4][nbase + 4 (i % 4)], lane j receives
// [kbase + 0..3][nbase + j], i.e. four consecutive k of one column — two such
// reads form an MFMA operand fragment, so NN and TN need no register
// transposes. K must be a multiple of BK; rows and columns past M / N are
// clamped on load (they only feed outputs that are not stored).
typedef short s16x4_t __attribute__((ext_vector_type(4)));

// The direct loads set M0 (the LDS destination) in inline assembly and list
// it as clobbered; clang warns that M0 is a reserved register. No code the
// compiler generates in these kernels keeps a value in M0 (the gfx950 LDS
// instructions they use do not read it), which the generated assembly shows.
#pragma clang diagnostic ignored "-Winline-asm"

#ifndef ORMI_GEMM_SCHED
#define ORMI_GEMM_SCHED 1
#endif

template <int BK>
__device__ __forceinline__ int swz_k(int r) {
    static_assert(BK == 32 || BK == 64, "tile depth 32 or 64");
    return BK == 64 ? (r & 7) ^ ((r >> 3) & 1) : ((r >> 1) & 3) ^ ((r >> 3) & 1);
}
__device__ __forceinline__ int swz_mn(int k) { return (k & 3) << 2; }

// Direct loads of one operand's BK-deep k-tiles into LDS. The per-lane byte
// offsets within a tile do not change along k, so they are computed once;
// each k-tile then costs one scalar base update and one load instruction
// per 1 KB segment (global_load_lds_dwordx4 with a scalar base and a 32-bit
// per-lane offset; the host keeps tile spans under 4 GB).
// KC: k-contiguous; BMN: tile extent along m (or n); NW: waves sharing the work.
template <int BMN, bool KC, int NW, int BK = 64>
struct DmaPlan {
    static constexpr int SEGS = BMN * BK * 2 / 1024;  // 1 KB segments per tile
    static constexpr int PER = SEGS / NW;
    static_assert(SEGS % NW == 0, "segments must split evenly over waves");
    unsigned voff[PER];

    // Rows and columns past MN are clamped (they only feed outputs that are
    // not stored); mn0 < MN, and for the mn-contiguous layout MN % 8 == 0.
    __device__ __forceinline__ void init(long long s_mn, long long s_k, int mn0, int MN) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
        for (int s = 0; s < PER; ++s) {
            const int q = wave * PER + s;
            if constexpr (KC) {
                constexpr int CPR = BK / 8;     // 16-byte chunks per row
                const int row = q * (64 / CPR) + lane / CPR;
                const int c = (lane % CPR) ^ swz_k<BK>(row);
                const int mn = min(mn0 + row, MN - 1) - mn0;
                voff[s] = (unsigned)(((long long)mn * s_mn + c * 8) * 2);
            } else {
                constexpr int CPR = BMN / 8;   // 16-byte chunks per k-row
                constexpr int RPS = 64 / CPR;  // k-rows per segment
                const int row = q * RPS + lane / CPR;
                const int c = (lane % CPR) ^ swz_mn(row);
                const int mn = min(mn0 + c * 8, MN - 8) - mn0;
                voff[s] = (unsigned)(((long long)row * s_k + mn) * 2);
            }
        }
    }
    // Byte offset of element (mn0, k0) from the operand base, and the step
    // between consecutive k-tiles.
    __device__ __forceinline__ static long long origin(long long s_mn, long long s_k, int mn0, int k0) {
        return KC ? ((long long)mn0 * s_mn + k0) * 2 : ((long long)k0 * s_k + mn0) * 2;
    }
    __device__ __forceinline__ static long long kstep(long long s_k) { return KC ? 2 * BK : 2 * BK * s_k; }

    // Issued as inline assembly: the compiler's wait-count pass assumes any
    // LDS read may alias a pending LDS DMA and would make every fragment read
    // of the current stage wait for these loads of the next stage. The kernel
    // waits for them itself (an explicit vmcnt before the barrier that
    // publishes a stage).
    // One load instruction (segment s of this wave's share) from a tile base
    // that is already uniform (in scalar registers).
    __device__ __forceinline__ void issue_one(lds_char* lds, const char* base, int s) const {
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const unsigned dst = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds + (wave * PER + s) * 1024));
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"(voff[s]), "s"(base)
                     : "memory", "m0");
    }
    __device__ __forceinline__ static const char* uniform(const char* tile) {
        const unsigned long long t = (unsigned long long)(uintptr_t)tile;
        const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)t);
        const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(t >> 32));
        return (const char*)(((unsigned long long)hi << 32) | lo);
    }

    __device__ __forceinline__ void issue(lds_char* lds, const char* tile) const {
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const unsigned long long t = (unsigned long long)(uintptr_t)tile;
        const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)t);
        const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(t >> 32));
        const char* base = (const char*)(((unsigned long long)hi << 32) | lo);
#pragma unroll
        for (int s = 0; s < PER; ++s) {
            const unsigned dst =
                __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds + (wave * PER + s) * 1024));
            asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"(voff[s]), "s"(base)
                         : "memory", "m0");
        }
    }
};

// MFMA operand fragment for tile rows [row0, row0 + 32) and k-step ks (16 k):
// lane l holds 8 consecutive k of row row0 + l % 32, starting at 16 ks + 8 (l / 32).
template <int BMN, bool KC, int BK = 64>
__device__ __forceinline__ u32x4_t frag(const lds_char* lds, int row0, int ks) {
    const int lane = threadIdx.x & 63;
    if constexpr (KC) {
        const int row = row0 + (lane & 31);
        const int c = ks * 2 + (lane >> 5);
        return *(const __attribute__((address_space(3))) u32x4_t*)(lds + row * (2 * BK) + ((c ^ swz_k<BK>(row)) << 4));
    } else {
        const int g = lane >> 4, i = lane & 15;
        const int nb = row0 + (g & 1) * 16 + 4 * (i & 3);
        u32x4_t out;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = ks * 16 + (g >> 1) * 8 + h * 4 + (i >> 2);
            const int c = nb >> 3;
            const lds_char* p = lds + k * (BMN * 2) + ((c ^ swz_mn(k)) << 4) + ((nb & 4) << 1);
            const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)p);
            out[2 * h] = (unsigned)(unsigned short)v[0] | ((unsigned)(unsigned short)v[1] << 16);
            out[2 * h + 1] = (unsigned)(unsigned short)v[2] | ((unsigned)(unsigned short)v[3] << 16);
        }
        return out;
    }
}

// One k-tile: run the MFMAs on this stage (As, Bs) while the next tile loads
// into the other stage (An, Bn), then wait for the loads and synchronize.
// The first fragments of this stage are requested before the loads are
// issued, so the LDS read latency of the tile's first step overlaps them.
template <typename Tr, int BM, int BN, int WGM, int WGN, bool A_KC, bool B_KC>
struct DmaStep {
    static constexpr int NW = WGM * WGN, BK = 64;
    static constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
    using PlanA = DmaPlan<BM, A_KC, NW>;
    using PlanB = DmaPlan<BN, B_KC, NW>;

    __device__ __forceinline__ static void run(const lds_char* As, const lds_char* Bs, lds_char* An, lds_char* Bn,
                                               bool load_next, const PlanA& pa, const PlanB& pb, const char* ta,
                                               const char* tb, int wm, int wn, f32x16_t (&acc)[TM][TN]) {
        u32x4_t af[2][TM], bfr[2][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) af[0][i] = frag<BM, A_KC>(As, wm * WTM + i * 32, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) bfr[0][j] = frag<BN, B_KC>(Bs, wn * WTN + j * 32, 0);
        if (load_next) {
            pa.issue(An, ta);
            pb.issue(Bn, tb);
        }
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int q = ks & 1;
            // Fragments of step ks+1 are requested before step ks's MFMAs
            // issue, so their LDS latency hides behind the matrix work; the
            // scheduling barriers keep the compiler from sinking the reads.
            if (ks + 1 < BK / 16) {
#pragma unroll
                for (int i = 0; i < TM; ++i) af[q ^ 1][i] = frag<BM, A_KC>(As, wm * WTM + i * 32, ks + 1);
#pragma unroll
                for (int j = 0; j < TN; ++j) bfr[q ^ 1][j] = frag<BN, B_KC>(Bs, wn * WTN + j * 32, ks + 1);
            }
            if (ORMI_GEMM_SCHED) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) Tr::mma(af[q][i], bfr[q][j], acc[i][j]);
            if (ORMI_GEMM_SCHED) __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }
};

template <typename Tr, int BM, int BN, int WGM, int WGN, bool A_KC, bool B_KC>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_dma_kernel(GemmParams p) {
    constexpr int NW = WGM * WGN, BK = 64;
    constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
    constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
    // Two stages in four distinct arrays.
    __shared__ __attribute__((aligned(1024))) char sa0[A_BYTES];
    __shared__ __attribute__((aligned(1024))) char sb0[B_BYTES];
    __shared__ __attribute__((aligned(1024))) char sa1[A_BYTES];
    __shared__ __attribute__((aligned(1024))) char sb1[B_BYTES];

    const int T = p.tiles_m * p.tiles_n;
    int t = blockIdx.x;
    if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
    constexpr int GROUP = 4;
    const int group_size = GROUP * p.tiles_n;
    const int g = t / group_size, first_m = g * GROUP;
    const int gm = min(p.tiles_m - first_m, GROUP);
    const int m0 = (first_m + (t % group_size) % gm) * BM;
    const int n0 = ((t % group_size) / gm) * BN;

    const int split = blockIdx.z % p.splits;
    int bidx = blockIdx.z / p.splits;
    long long a_off = 0, b_off = 0;
    const long long c_off = ((long long)split * p.batch + bidx) * p.M * p.N;
    for (int d = p.batch_ndim - 1; d >= 0; --d) {
        const int coord = bidx % p.batch_shape[d];
        bidx /= p.batch_shape[d];
        a_off += coord * p.a_bs[d];
        b_off += coord * p.b_bs[d];
    }
    float* c = p.c + c_off;
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int KT = kend > kbeg ? (kend - kbeg) / BK : 0;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

    using Step = DmaStep<Tr, BM, BN, WGM, WGN, A_KC, B_KC>;
    typename Step::PlanA pa;
    typename Step::PlanB pb;
    pa.init(p.a_sm, p.a_sk, m0, p.M);
    pb.init(p.b_sn, p.b_sk, n0, p.N);
    const char* ta = p.a + a_off * 2 + Step::PlanA::origin(p.a_sm, p.a_sk, m0, kbeg);
    const char* tb = p.b + b_off * 2 + Step::PlanB::origin(p.b_sn, p.b_sk, n0, kbeg);
    const long long a_step = Step::PlanA::kstep(p.a_sk), b_step = Step::PlanB::kstep(p.b_sk);

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if (KT > 0) {
        pa.issue((lds_char*)sa0, ta);
        pb.issue((lds_char*)sb0, tb);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const bool odd = kt & 1;
        lds_char* A0 = (lds_char*)sa0;
        lds_char* A1 = (lds_char*)sa1;
        lds_char* B0 = (lds_char*)sb0;
        lds_char* B1 = (lds_char*)sb1;
        ta += a_step;
        tb += b_step;
        Step::run(odd ? A1 : A0, odd ? B1 : B0, odd ? A0 : A1, odd ? B0 : B1, kt + 1 < KT, pa, pb, ta, tb, wm, wn, acc);
    }

#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < p.M && col < p.N) c[(long long)row * p.N + col] = acc[i][j][r];
            }
        }
    }
}

// Second pass after a K split, or after a kernel that has no epilogue of its
// own: v = sum over splits q (in order) of ws[q][b][m][n], then the epilogue
// (or a plain store). Rows of all batches run along grid y; each thread takes
// 4 consecutive columns of a row, issuing all its loads (16-byte ones when
// VEC: N % 4 == 0 and C, aux 16-byte aligned) before its stores.
struct FinishParams {
    float* c;
    const float* ws;
    long long n;  // elements per split: batch * M * N
    int splits, M, N, rows;  // rows = batch * M
    int batch_ndim;
    int batch_shape[ORMI_GEMM_MAX_BATCH_DIMS];
    Epi epi;
};

template <bool VEC>
__global__ __launch_bounds__(256) void gemm_finish_kernel(FinishParams f) {
    const Epi& e = f.epi;
    const float sv = e.s ? *e.s : 0.0f;
    const bool reads_d = epi_reads_d(e);
    for (int row = blockIdx.y; row < f.rows; row += gridDim.y) {
        const int bi = row / f.M, m = row - bi * f.M;
        long long d_off = 0;
        if (reads_d) {
            int rest = bi;
            for (int d = f.batch_ndim - 1; d >= 0; --d) {
                d_off += (long long)(rest % f.batch_shape[d]) * e.d_bs[d];
                rest /= f.batch_shape[d];
            }
            d_off += (long long)m * e.d_sm;
        }
        const long long base = (long long)row * f.N;
        for (int col0 = (blockIdx.x * blockDim.x + threadIdx.x) * 4; col0 < f.N; col0 += gridDim.x * blockDim.x * 4) {
            const int cnt = min(4, f.N - col0);
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f}, dv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (reads_d) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (k < cnt) dv[k] = e.d[d_off + (long long)(col0 + k) * e.d_sn];
            }
            for (int q = 0; q < f.splits; ++q) {
                const float* w = f.ws + (long long)q * f.n + base + col0;
                float t[4];
                if (VEC) {
                    const ormi_f4 x = *(const ormi_f4*)w;
#pragma unroll
                    for (int k = 0; k < 4; ++k) t[k] = x[k];
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) t[k] = k < cnt ? w[k] : 0.0f;
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) v[k] = q == 0 ? t[k] : v[k] + t[k];
            }
            if (VEC && e.kind == ORMI_GEMM_EPI_NONE) {
                *(ormi_f4*)(f.c + base + col0) = ormi_f4{v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (k < cnt) epi_store(e, sv, f.c, e.aux, base + col0 + k, dv[k], v[k]);
            }
        }
    }
}

// The finish pass without an epilogue, for C contiguous over the n elements
// of a split and 16-byte aligned (n % 4 == 0): a flat grid-stride walk over
// float4 groups, U groups per thread with every split's loads issued before
// the sums, in split order like gemm_finish_kernel.
template <int U>
__global__ __launch_bounds__(256) void gemm_finish_flat_kernel(float* __restrict__ c, const float* __restrict__ ws,
                                                               long long n4, int splits) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    const ormi_f4* w = (const ormi_f4*)ws;
    ormi_f4* out = (ormi_f4*)c;
    for (long long g0 = (long long)blockIdx.x * blockDim.x + threadIdx.x; g0 < n4; g0 += stride * U) {
        ormi_f4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long g = g0 + u * stride;
            if (g < n4) v[u] = w[g];
        }
        for (int q = 1; q < splits; ++q) {
            ormi_f4 t[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const long long g = g0 + u * stride;
                if (g < n4) t[u] = w[q * n4 + g];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] += t[u];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long g = g0 + u * stride;
            if (g < n4) __builtin_nontemporal_store(v[u], out + g);
        }
    }
}

// Operand packing for the GEMMs the fast kernels cannot take as given (a
// unit-stride extent or another stride not in whole 16-byte chunks, an
// unaligned base): the operand, rows mn < MN by depth k < K with any element
// strides and batch strides, is copied into a dense k-contiguous buffer
// [batch][MN][K_pad] (K_pad a multiple of 64), zero for k >= K, so the product
// over K_pad equals the one over K exactly. One 64 x 64 block per work-group;
// an mn-contiguous source is read along mn and transposed through LDS, any
// other along k.
struct PackParams {
    long long s_mn, s_k;
    int MN, K, K_pad;
    int batch_ndim;
    int batch_shape[ORMI_GEMM_MAX_BATCH_DIMS];
    long long bs[ORMI_GEMM_MAX_BATCH_DIMS];
};

template <typename T, bool MN_UNIT>
__global__ __launch_bounds__(256) void gemm_pack_kernel(T* __restrict__ dst, const T* __restrict__ src, PackParams pp) {
    const int k0 = blockIdx.x * 64, mn0 = blockIdx.y * 64;
    long long boff = 0;
    int rest = blockIdx.z;
    for (int d = pp.batch_ndim - 1; d >= 0; --d) {
        boff += (long long)(rest % pp.batch_shape[d]) * pp.bs[d];
        rest /= pp.batch_shape[d];
    }
    const T* s = src + boff;
    T* o = dst + (long long)blockIdx.z * pp.MN * pp.K_pad;
    if constexpr (MN_UNIT) {
        __shared__ T tile[64][65];
        for (int i = threadIdx.x; i < 64 * 64; i += 256) {
            const int kk = i >> 6, mm = i & 63, k = k0 + kk, mn = mn0 + mm;
            tile[kk][mm] = (k < pp.K && mn < pp.MN) ? s[(long long)k * pp.s_k + mn] : T(0);
        }
        __syncthreads();
        for (int i = threadIdx.x; i < 64 * 64; i += 256) {
            const int mm = i >> 6, kk = i & 63, k = k0 + kk, mn = mn0 + mm;
            if (mn < pp.MN) o[(long long)mn * pp.K_pad + k] = tile[kk][mm];
        }
    } else {
        for (int i = threadIdx.x; i < 64 * 64; i += 256) {
            const int mm = i >> 6, kk = i & 63, k = k0 + kk, mn = mn0 + mm;
            if (mn < pp.MN) o[(long long)mn * pp.K_pad + k] = k < pp.K ? s[(long long)mn * pp.s_mn + (long long)k * pp.s_k] : T(0);
        }
    }
}

// Any strides, any shape: 16x16 output tile per block, fp32 accumulation.
template <int DT>
__device__ __forceinline__ float gemm_elem(const void* p, long long i) {
    if constexpr (DT == ORMI_DTYPE_F32) return ((const float*)p)[i];
    else if constexpr (DT == ORMI_DTYPE_BF16) return __uint_as_float((unsigned)((const unsigned short*)p)[i] << 16);
    else {
        const unsigned short h = ((const unsigned short*)p)[i];
        _Float16 x;
        __builtin_memcpy(&x, &h, 2);
        return (float)x;
    }
}

template <int DT>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmParams p) {
    __shared__ float As[16][17];
    __shared__ float Bs[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;
    long long a_off = 0, b_off = 0, d_off = 0;
    int bidx = blockIdx.z;
    const long long c_off = (long long)bidx * p.M * p.N;
    for (int d = p.batch_ndim - 1; d >= 0; --d) {
        const int coord = bidx % p.batch_shape[d];
        bidx /= p.batch_shape[d];
        a_off += coord * p.a_bs[d];
        b_off += coord * p.b_bs[d];
        d_off += coord * p.epi.d_bs[d];
    }
    float acc = 0.0f;
    for (int k0 = 0; k0 < p.K; k0 += 16) {
        const int ar = blockIdx.y * 16 + ty, ak = k0 + tx;
        const int bk = k0 + ty, bc = blockIdx.x * 16 + tx;
        As[ty][tx] = (ar < p.M && ak < p.K) ? gemm_elem<DT>(p.a, a_off + (long long)ar * p.a_sm + (long long)ak * p.a_sk) : 0.0f;
        Bs[ty][tx] = (bk < p.K && bc < p.N) ? gemm_elem<DT>(p.b, b_off + (long long)bk * p.b_sk + (long long)bc * p.b_sn) : 0.0f;
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) acc = __builtin_fmaf(As[ty][kk], Bs[kk][tx], acc);
        __syncthreads();
    }
    if (row < p.M && col < p.N) {
        const Epi& e = p.epi;
        const float dv = epi_reads_d(e) ? e.d[d_off + row * e.d_sm + col * e.d_sn] : 0.0f;
        epi_store(e, e.s ? *e.s : 0.0f, p.c + c_off, e.aux ? e.aux + c_off : nullptr, (long long)row * p.N + col, dv, acc);
    }
}

// ------------------------------------------------------------------ dispatch --
struct Cfg {
    int BM, BN, BK;
};

template <typename Tr, int BM, int BN, int BK, int WGM, int WGN>
struct Launcher {
    static constexpr Cfg cfg{BM, BN, BK};
    template <bool A_KC, bool B_KC>
    static void go(const GemmParams& p, dim3 grid, bool even) {
        if (even) gemm_mfma_kernel<Tr, BM, BN, BK, WGM, WGN, A_KC, B_KC, true><<<grid, 64 * WGM * WGN>>>(p);
        else gemm_mfma_kernel<Tr, BM, BN, BK, WGM, WGN, A_KC, B_KC, false><<<grid, 64 * WGM * WGN>>>(p);
    }
    static void run(const GemmParams& p, dim3 grid, bool even, bool a_kc, bool b_kc) {
        if (a_kc && b_kc) go<true, true>(p, grid, even);
        else if (a_kc) go<true, false>(p, grid, even);
        else if (b_kc) go<false, true>(p, grid, even);
        else go<false, false>(p, grid, even);
    }
};

// 16-bit configurations, selectable with ORMI_GEMM_CFG16 for tuning:
//   0: 256x256x64, 2x2 waves (128x128 per wave, 1 wave/SIMD)
//   1: 256x256x64, 2x4 waves (128x64 per wave, 2 waves/SIMD)
//   2: 256x256x64, 4x2 waves (64x128 per wave, 2 waves/SIMD)
//   3: 128x128x64, 2x2 waves (64x64 per wave, 2 blocks/CU)
// fp32 configurations (ORMI_GEMM_CFG32 forces one; by default 2 for shapes in
// whole 128x256 tiles, and 3 for short-K shapes that 128x256 tiles cannot
// spread over the CUs and for shapes with partial tiles):
//   0: 128x128x32, 2x2 waves (64x64 per wave)
//   1: 256x128x32, 4x2 waves (64x64 per wave)
//   2: 128x256x32, 2x4 waves (64x64 per wave)
//   3: 128x128x32, 2x4 waves (64x32 per wave)
//   4: 128x128x32, 4x2 waves (32x64 per wave)
static int env_cfg(const char* name, int dflt) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : dflt;
}

template <typename Tr>
static Cfg cfg16(int id) {
    switch (id) {
        case 0: return Launcher<Tr, 256, 256, 64, 2, 2>::cfg;
        case 1: return Launcher<Tr, 256, 256, 64, 2, 4>::cfg;
        case 2: return Launcher<Tr, 256, 256, 64, 4, 2>::cfg;
        default: return Launcher<Tr, 128, 128, 64, 2, 2>::cfg;
    }
}
template <typename Tr>
static void run16(int id, const GemmParams& p, dim3 grid, bool even, bool a_kc, bool b_kc) {
    switch (id) {
        case 0: Launcher<Tr, 256, 256, 64, 2, 2>::run(p, grid, even, a_kc, b_kc); break;
        case 1: Launcher<Tr, 256, 256, 64, 2, 4>::run(p, grid, even, a_kc, b_kc); break;
        case 2: Launcher<Tr, 256, 256, 64, 4, 2>::run(p, grid, even, a_kc, b_kc); break;
        default: Launcher<Tr, 128, 128, 64, 2, 2>::run(p, grid, even, a_kc, b_kc); break;
    }
}
static Cfg cfg32(int id) {
    switch (id) {
        case 1: return Launcher<TrF32, 256, 128, 32, 4, 2>::cfg;
        case 2: return Launcher<TrF32, 128, 256, 32, 2, 4>::cfg;
        case 3: return Launcher<TrF32, 128, 128, 32, 2, 4>::cfg;
        case 4: return Launcher<TrF32, 128, 128, 32, 4, 2>::cfg;
        default: return Launcher<TrF32, 128, 128, 32, 2, 2>::cfg;
    }
}
static void run32(int id, const GemmParams& p, dim3 grid, bool even, bool a_kc, bool b_kc) {
    switch (id) {
        case 1: Launcher<TrF32, 256, 128, 32, 4, 2>::run(p, grid, even, a_kc, b_kc); break;
        case 2: Launcher<TrF32, 128, 256, 32, 2, 4>::run(p, grid, even, a_kc, b_kc); break;
        case 3: Launcher<TrF32, 128, 128, 32, 2, 4>::run(p, grid, even, a_kc, b_kc); break;
        case 4: Launcher<TrF32, 128, 128, 32, 4, 2>::run(p, grid, even, a_kc, b_kc); break;
        default: Launcher<TrF32, 128, 128, 32, 2, 2>::run(p, grid, even, a_kc, b_kc); break;
    }
}

// ------------------------------------------------------------------------
// Multi-stage direct-load GEMM. STAGES k-tiles of depth BK live in LDS; the
// loads of tile kt + STAGES - 1 are issued while tile kt is multiplied, so
// each tile's loads have STAGES - 2 tiles plus half a tile of matrix work to
// arrive (LDS holds STAGES tiles; at 256x256x32, 4 stages use 128 KB).
//
// Per tile (KS = BK / 16 MFMA k-steps, fragments double-buffered in registers):
//   ks < KS-1 : read fragments of step ks+1, MFMAs of step ks;
//   ks = KS-1 : wait until this wave's loads of tile kt+1 have landed (vmcnt),
//               barrier (every wave's loads of kt+1 landed, every wave done
//               with tile kt-1's stage), issue the loads of tile kt+STAGES-1
//               into that freed stage, read step 0 of tile kt+1, MFMAs of
//               step KS-1.
// One barrier per tile; the loads are counted per wave (PER instructions per
// operand per tile), so the vmcnt bound is exact.
// Wait until at most n tiles' loads (PER_TILE instructions each) are pending.
template <int PER_TILE, int MAXN>
__device__ __forceinline__ void wait_tiles(int n) {
    if constexpr (MAXN >= 3) { if (n >= 3) { wait_vmcnt<3 * PER_TILE>(); return; } }
    if constexpr (MAXN >= 2) { if (n >= 2) { wait_vmcnt<2 * PER_TILE>(); return; } }
    if constexpr (MAXN >= 1) { if (n >= 1) { wait_vmcnt<PER_TILE>(); return; } }
    wait_vmcnt<0>();
}

template <typename Tr, int BM, int BN, int BK, int WGM, int WGN, int STAGES, bool A_KC, bool B_KC>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_pipe_kernel(GemmParams p) {
    static_assert(STAGES >= 3 && STAGES <= 5, "3 to 5 stages");
    constexpr int NW = WGM * WGN, KS = BK / 16;
    static_assert(KS % 2 == 0, "fragment buffers alternate per k-step");
    constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
    constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2, STAGE = A_BYTES + B_BYTES;
    __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE];
    using PlanA = DmaPlan<BM, A_KC, NW, BK>;
    using PlanB = DmaPlan<BN, B_KC, NW, BK>;
    constexpr int PER_TILE = PlanA::PER + PlanB::PER;

    const int T = p.tiles_m * p.tiles_n;
    int t = blockIdx.x;
    if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
    constexpr int GROUP = 4;
    const int group_size = GROUP * p.tiles_n;
    const int g = t / group_size, first_m = g * GROUP;
    const int gm = min(p.tiles_m - first_m, GROUP);
    const int m0 = (first_m + (t % group_size) % gm) * BM;
    const int n0 = ((t % group_size) / gm) * BN;

    const int split = blockIdx.z % p.splits;
    int bidx = blockIdx.z / p.splits;
    long long a_off = 0, b_off = 0;
    const long long c_off = ((long long)split * p.batch + bidx) * p.M * p.N;
    for (int d = p.batch_ndim - 1; d >= 0; --d) {
        const int coord = bidx % p.batch_shape[d];
        bidx /= p.batch_shape[d];
        a_off += coord * p.a_bs[d];
        b_off += coord * p.b_bs[d];
    }
    float* c = p.c + c_off;
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int KT = kend > kbeg ? (kend - kbeg) / BK : 0;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

    PlanA pa;
    PlanB pb;
    pa.init(p.a_sm, p.a_sk, m0, p.M);
    pb.init(p.b_sn, p.b_sk, n0, p.N);
    const char* ta = p.a + a_off * 2 + PlanA::origin(p.a_sm, p.a_sk, m0, kbeg);
    const char* tb = p.b + b_off * 2 + PlanB::origin(p.b_sn, p.b_sk, n0, kbeg);
    const long long a_step = PlanA::kstep(p.a_sk), b_step = PlanB::kstep(p.b_sk);
    lds_char* const lds = (lds_char*)smem;
    // Kernel arguments the epilogue needs are loaded here: a scalar load still
    // in flight when the loop starts would make every LDS wait in the loop
    // drain completely (scalar loads return out of order, so the wait-count
    // pass can no longer count LDS reads precisely).
    asm volatile("" ::"s"(c), "s"(p.M), "s"(p.N));

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Prologue: tiles 0 .. STAGES-2 into stages 0 .. STAGES-2.
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) {
        if (s < KT) {
            pa.issue(lds + s * STAGE, ta);
            pb.issue(lds + s * STAGE + A_BYTES, tb);
            ta += a_step;
            tb += b_step;
        }
    }
    int issued = min(KT, STAGES - 1);  // tiles whose loads have been issued
    u32x4_t af[2][TM], bfr[2][TN];
    if (KT > 0) {
        wait_tiles<PER_TILE, STAGES - 2>(issued - 1);
        lds_barrier();
#pragma unroll
        for (int i = 0; i < TM; ++i) af[0][i] = frag<BM, A_KC, BK>(lds, wm * WTM + i * 32, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) bfr[0][j] = frag<BN, B_KC, BK>(lds + A_BYTES, wn * WTN + j * 32, 0);
    }

    int stage = 0;
    for (int kt = 0; kt < KT; ++kt) {
        const lds_char* As = lds + stage * STAGE;
        const lds_char* Bs = As + A_BYTES;
        const int next_stage = stage + 1 == STAGES ? 0 : stage + 1;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int q = ks & 1;
            if (ks + 1 < KS) {
#pragma unroll
                for (int i = 0; i < TM; ++i) af[q ^ 1][i] = frag<BM, A_KC, BK>(As, wm * WTM + i * 32, ks + 1);
#pragma unroll
                for (int j = 0; j < TN; ++j) bfr[q ^ 1][j] = frag<BN, B_KC, BK>(Bs, wn * WTN + j * 32, ks + 1);
            } else if (kt + 1 < KT) {
                // Tiles issued after kt+1 may stay in flight.
                wait_tiles<PER_TILE, STAGES - 3>(issued - (kt + 2));
                lds_barrier();
                if (issued < KT) {
                    // The freed stage is the one tile kt-1 used, i.e. (kt + STAGES - 1) % STAGES.
                    const int fs = next_stage + STAGES - 2 >= STAGES ? next_stage - 2 : next_stage + STAGES - 2;
                    pa.issue(lds + fs * STAGE, ta);
                    pb.issue(lds + fs * STAGE + A_BYTES, tb);
                    ta += a_step;
                    tb += b_step;
                    ++issued;
                }
                const lds_char* An = lds + next_stage * STAGE;
#pragma unroll
                for (int i = 0; i < TM; ++i) af[q ^ 1][i] = frag<BM, A_KC, BK>(An, wm * WTM + i * 32, 0);
#pragma unroll
                for (int j = 0; j < TN; ++j) bfr[q ^ 1][j] = frag<BN, B_KC, BK>(An + A_BYTES, wn * WTN + j * 32, 0);
            }
            if (ORMI_GEMM_SCHED) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) Tr::mma(af[q][i], bfr[q][j], acc[i][j]);
            if (ORMI_GEMM_SCHED) __builtin_amdgcn_sched_barrier(0);
        }
        stage = next_stage;
    }

#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < p.M && col < p.N) c[(long long)row * p.N + col] = acc[i][j][r];
            }
        }
    }
}

// ------------------------------------------------------------------------
// Interleaved multi-stage GEMM (BK 32, two MFMA k-steps per tile). Same LDS
// stages and direct loads as gemm_pipe_kernel, but each MFMA of a step is
// followed by a share of the step's memory instructions — the fragment reads
// of the next step, then half of the direct loads of tile kt + STAGES - 1 —
// in a fixed order, so the matrix pipe never waits on a burst of loads and
// every read is in flight while earlier MFMAs execute. Loads past the last
// tile re-read the last tile into a stage no step reads, which keeps the
// per-wave load count of every tile the same and every vmcnt bound a
// constant: the loop has no branches besides its own.
//   step 0: MFMAs on k-step 0 | reads of k-step 1 (this stage), loads 0..HALF-1
//   wait: this wave's loads of tile kt+1 landed, its LDS reads done; barrier
//   step 1: MFMAs on k-step 1 | reads of k-step 0 (next stage), loads HALF..
// The barrier publishes tile kt+1 and tells every wave that tile kt-1's
// stage, refilled during tile kt, has no reads left.
template <int BMN, bool KC, int BK>
__device__ __forceinline__ void frag_part(u32x4_t& f, const lds_char* lds, int row0, int ks, int h) {
    if constexpr (KC) {
        f = frag<BMN, true, BK>(lds, row0, ks);
    } else {
        const int lane = threadIdx.x & 63;
        const int g = lane >> 4, i = lane & 15;
        const int nb = row0 + (g & 1) * 16 + 4 * (i & 3);
        const int k = ks * 16 + (g >> 1) * 8 + h * 4 + (i >> 2);
        const lds_char* p = lds + k * (BMN * 2) + (((nb >> 3) ^ swz_mn(k)) << 4) + ((nb & 4) << 1);
        const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)p);
        f[2 * h] = (unsigned)(unsigned short)v[0] | ((unsigned)(unsigned short)v[1] << 16);
        f[2 * h + 1] = (unsigned)(unsigned short)v[2] | ((unsigned)(unsigned short)v[3] << 16);
    }
}

template <typename Tr, int BM, int BN, int WGM, int WGN, bool A_KC, bool B_KC>
struct IlStep {
    static constexpr int BK = 32, NW = WGM * WGN;
    static constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
    static constexpr int A_BYTES = BM * BK * 2;
    using PlanA = DmaPlan<BM, A_KC, NW, BK>;
    using PlanB = DmaPlan<BN, B_KC, NW, BK>;
    static constexpr int PA = PlanA::PER, PB = PlanB::PER, PER_TILE = PA + PB, HALF = PER_TILE / 2;
    static_assert(PER_TILE % 2 == 0, "loads split evenly over the two steps");
    static constexpr int RA = A_KC ? 1 : 2, RB = B_KC ? 1 : 2;  // reads per fragment
    static constexpr int NR = TM * RA + TN * RB;                // reads per step
    static constexpr int NO = NR + HALF;                        // memory instructions per step
    static constexpr int NM = TM * TN;                          // MFMAs per step

    // Memory instruction o of a step. Reads come in the order the next step's
    // MFMAs consume them: A0, B0 .. B(TN-1), A1 .. A(TM-1).
    __device__ __forceinline__ static void mem_op(int o, int step, u32x4_t (&fa)[TM], u32x4_t (&fb)[TN],
                                                  const lds_char* rs, int rks, int wm, int wn, lds_char* fs,
                                                  const char* ta, const char* tb, const PlanA& pa, const PlanB& pb) {
        if (o < RA) {
            frag_part<BM, A_KC, BK>(fa[0], rs, wm * WTM, rks, o);
        } else if (o < RA + TN * RB) {
            const int j = (o - RA) / RB, h = (o - RA) % RB;
            frag_part<BN, B_KC, BK>(fb[j], rs + A_BYTES, wn * WTN + j * 32, rks, h);
        } else if (o < NR) {
            const int q = o - RA - TN * RB;
            const int i = 1 + q / RA, h = q % RA;
            frag_part<BM, A_KC, BK>(fa[i], rs, wm * WTM + i * 32, rks, h);
        } else {
            const int d = step * HALF + (o - NR);
            if (d < PA) pa.issue_one(fs, ta, d);
            else pb.issue_one(fs + A_BYTES, tb, d - PA);
        }
    }

    __device__ __forceinline__ static void run(int step, f32x16_t (&acc)[TM][TN], const u32x4_t (&ua)[TM],
                                               const u32x4_t (&ub)[TN], u32x4_t (&fa)[TM], u32x4_t (&fb)[TN],
                                               const lds_char* rs, int rks, int wm, int wn, lds_char* fs,
                                               const char* ta, const char* tb, const PlanA& pa, const PlanB& pb) {
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            Tr::mma(ua[n / TN], ub[n % TN], acc[n / TN][n % TN]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int o = n * NO / NM; o < (n + 1) * NO / NM; ++o) {
                mem_op(o, step, fa, fb, rs, rks, wm, wn, fs, ta, tb, pa, pb);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
};

template <typename Tr, int BM, int BN, int WGM, int WGN, int STAGES, bool A_KC, bool B_KC>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_il_kernel(GemmParams p) {
    static_assert(STAGES >= 3 && STAGES <= 5, "3 to 5 stages");
    using Step = IlStep<Tr, BM, BN, WGM, WGN, A_KC, B_KC>;
    constexpr int BK = Step::BK, TM = Step::TM, TN = Step::TN, WTM = Step::WTM, WTN = Step::WTN;
    constexpr int A_BYTES = Step::A_BYTES, STAGE = A_BYTES + BN * BK * 2;
    constexpr int PER_TILE = Step::PER_TILE, HALF = Step::HALF;
    __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE];

    const int T = p.tiles_m * p.tiles_n;
    int t = blockIdx.x;
    if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
    constexpr int GROUP = 4;
    const int group_size = GROUP * p.tiles_n;
    const int g = t / group_size, first_m = g * GROUP;
    const int gm = min(p.tiles_m - first_m, GROUP);
    const int m0 = (first_m + (t % group_size) % gm) * BM;
    const int n0 = ((t % group_size) / gm) * BN;

    const int split = blockIdx.z % p.splits;
    int bidx = blockIdx.z / p.splits;
    long long a_off = 0, b_off = 0;
    const long long c_off = ((long long)split * p.batch + bidx) * p.M * p.N;
    for (int d = p.batch_ndim - 1; d >= 0; --d) {
        const int coord = bidx % p.batch_shape[d];
        bidx /= p.batch_shape[d];
        a_off += coord * p.a_bs[d];
        b_off += coord * p.b_bs[d];
    }
    float* c = p.c + c_off;
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int KT = kend > kbeg ? (kend - kbeg) / BK : 0;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

    typename Step::PlanA pa;
    typename Step::PlanB pb;
    pa.init(p.a_sm, p.a_sk, m0, p.M);
    pb.init(p.b_sn, p.b_sk, n0, p.N);
    const char* ta = p.a + a_off * 2 + Step::PlanA::origin(p.a_sm, p.a_sk, m0, kbeg);
    const char* tb = p.b + b_off * 2 + Step::PlanB::origin(p.b_sn, p.b_sk, n0, kbeg);
    const long long a_step = Step::PlanA::kstep(p.a_sk), b_step = Step::PlanB::kstep(p.b_sk);
    lds_char* const lds = (lds_char*)smem;
    // Kernel arguments the epilogue needs are loaded here: a scalar load still
    // in flight when the loop starts would make every LDS wait in the loop
    // drain completely (scalar loads return out of order).
    asm volatile("" ::"s"(c), "s"(p.M), "s"(p.N));

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if (KT > 0) {
        // Prologue: tiles 0 .. STAGES-2 (a tile past the end re-reads the last one).
        // ta / tb always address tile min(next tile to load, KT - 1).
#pragma unroll
        for (int s = 0; s < STAGES - 1; ++s) {
            pa.issue(lds + s * STAGE, ta);
            pb.issue(lds + s * STAGE + A_BYTES, tb);
            if (s + 1 < KT) {
                ta += a_step;
                tb += b_step;
            }
        }
        wait_vmcnt<(STAGES - 2) * PER_TILE>();
        lds_barrier();
        u32x4_t fa[2][TM], fb[2][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[0][i] = frag<BM, A_KC, BK>(lds, wm * WTM + i * 32, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[0][j] = frag<BN, B_KC, BK>(lds + A_BYTES, wn * WTN + j * 32, 0);

        int stage = 0, free_stage = STAGES - 1;
        for (int kt = 0; kt < KT; ++kt) {
            const int next = stage + 1 == STAGES ? 0 : stage + 1;
            const lds_char* cur = lds + stage * STAGE;
            lds_char* fs = lds + free_stage * STAGE;
            const char* ua = Step::PlanA::uniform(ta);
            const char* ub = Step::PlanB::uniform(tb);
            Step::run(0, acc, fa[0], fb[0], fa[1], fb[1], cur, 1, wm, wn, fs, ua, ub, pa, pb);
            // vmcnt: loads issued after tile kt+1 (STAGES-3 whole tiles and half
            // of tile kt+STAGES-1) may stay in flight; lgkmcnt(0): own reads done.
            constexpr int V = (STAGES - 3) * PER_TILE + HALF;
            __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | (7 << 4));
            lds_barrier();
            Step::run(1, acc, fa[1], fb[1], fa[0], fb[0], lds + next * STAGE, 0, wm, wn, fs, ua, ub, pa, pb);
            if (kt + STAGES < KT) {
                ta += a_step;
                tb += b_step;
            }
            stage = next;
            free_stage = free_stage + 1 == STAGES ? 0 : free_stage + 1;
        }
        // No load may still be writing this workgroup's LDS when it exits.
        wait_vmcnt<0>();
    }

#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < p.M && col < p.N) c[(long long)row * p.N + col] = acc[i][j][r];
            }
        }
    }
}

// ------------------------------------------------------------------------
// Interleaved GEMM with whole-line loads of a k-contiguous A. In a 32-deep
// k-tile each row of a k-contiguous operand is 64 bytes, half a cache line,
// so every direct load of gemm_il_kernel touches 16 half lines. Here A is
// loaded 64 k deep: 8 rows of one whole 128-byte line per load instruction.
// A sits in 3 pair slots of 32 KB ([BM rows][64 k], the BK-64 swizzle), B in
// 4 slots of 16 KB as in gemm_il_kernel: 160 KB. Pair q (k-tiles 2q, 2q+1) is
// loaded half per k-tile during k-tiles 2q-4 and 2q-3, into the slot of pair
// q-3, whose last reads completed at the barrier of k-tile 2q-5; B k-tile
// kt+3 is loaded during kt into the slot of kt-1. Per k-tile kt:
//   step 0: MFMAs on k-step 0 | reads of k-step 1, A loads (half kt & 1 of pair kt/2 + 2)
//   wait: loads of k-tile kt-2 and older landed, own reads done; barrier
//   step 1: MFMAs on k-step 1 | reads of k-step 0 of kt+1, B loads (k-tile kt+3)
// Loads past the end re-read the last pair or tile into a slot no step reads,
// so every vmcnt bound is a constant. K must be a multiple of 64.
template <typename Tr, int BM, int BN, int WGM, int WGN, bool B_KC>
struct IlpStep {
    static constexpr int NW = WGM * WGN;
    static constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
    static constexpr int A_SLOT = BM * 64 * 2, B_SLOT = BN * 32 * 2;
    using PlanA = DmaPlan<BM, true, NW, 64>;
    using PlanB = DmaPlan<BN, B_KC, NW, 32>;
    static constexpr int PA = PlanA::PER / 2, PB = PlanB::PER;  // loads per step
    static_assert(PA == PB, "both steps issue the same number of loads");
    static constexpr int RB = B_KC ? 1 : 2;
    static constexpr int NR = TM + TN * RB;  // reads per step
    static constexpr int NO = NR + PA;       // memory instructions per step
    static constexpr int NM = TM * TN;       // MFMAs per step

    // Memory instruction o of step S: reads in the order the next step's MFMAs
    // consume them (A0, B0 .. B(TN-1), A1 .. A(TM-1)), then the loads.
    template <int S, int H>
    __device__ __forceinline__ static void mem_op(int o, u32x4_t (&fa)[TM], u32x4_t (&fb)[TN], const lds_char* ra,
                                                  int aks, const lds_char* rb, int bks, int wm, int wn, lds_char* la,
                                                  lds_char* lb, const char* ta, const char* tb, const PlanA& pa,
                                                  const PlanB& pb) {
        if (o < 1) {
            fa[0] = frag<BM, true, 64>(ra, wm * WTM, aks);
        } else if (o < 1 + TN * RB) {
            const int j = (o - 1) / RB, h = (o - 1) % RB;
            frag_part<BN, B_KC, 32>(fb[j], rb, wn * WTN + j * 32, bks, h);
        } else if (o < NR) {
            const int i = 1 + (o - 1 - TN * RB);
            fa[i] = frag<BM, true, 64>(ra, wm * WTM + i * 32, aks);
        } else if (S == 0) {
            pa.issue_one(la, ta, H * PA + (o - NR));
        } else {
            pb.issue_one(lb, tb, o - NR);
        }
    }

    template <int S, int H>
    __device__ __forceinline__ static void run(f32x16_t (&acc)[TM][TN], const u32x4_t (&ua)[TM], const u32x4_t (&ub)[TN],
                                               u32x4_t (&fa)[TM], u32x4_t (&fb)[TN], const lds_char* ra, int aks,
                                               const lds_char* rb, int bks, int wm, int wn, lds_char* la, lds_char* lb,
                                               const char* ta, const char* tb, const PlanA& pa, const PlanB& pb) {
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            Tr::mma(ua[n / TN], ub[n % TN], acc[n / TN][n % TN]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int o = n * NO / NM; o < (n + 1) * NO / NM; ++o) {
                mem_op<S, H>(o, fa, fb, ra, aks, rb, bks, wm, wn, la, lb, ta, tb, pa, pb);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
};

template <typename Tr, int BM, int BN, int WGM, int WGN, bool B_KC>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_ilp_kernel(GemmParams p) {
    using Step = IlpStep<Tr, BM, BN, WGM, WGN, B_KC>;
    constexpr int TM = Step::TM, TN = Step::TN, WTM = Step::WTM, WTN = Step::WTN;
    constexpr int A_SLOT = Step::A_SLOT, B_SLOT = Step::B_SLOT, PA = Step::PA;
    constexpr int A_SLOTS = 3, B_SLOTS = 4;
    __shared__ __attribute__((aligned(1024))) char smem[A_SLOTS * A_SLOT + B_SLOTS * B_SLOT];

    const int T = p.tiles_m * p.tiles_n;
    int t = blockIdx.x;
    if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
    constexpr int GROUP = 4;
    const int group_size = GROUP * p.tiles_n;
    const int g = t / group_size, first_m = g * GROUP;
    const int gm = min(p.tiles_m - first_m, GROUP);
    const int m0 = (first_m + (t % group_size) % gm) * BM;
    const int n0 = ((t % group_size) / gm) * BN;

    const int split = blockIdx.z % p.splits;
    int bidx = blockIdx.z / p.splits;
    long long a_off = 0, b_off = 0;
    const long long c_off = ((long long)split * p.batch + bidx) * p.M * p.N;
    for (int d = p.batch_ndim - 1; d >= 0; --d) {
        const int coord = bidx % p.batch_shape[d];
        bidx /= p.batch_shape[d];
        a_off += coord * p.a_bs[d];
        b_off += coord * p.b_bs[d];
    }
    float* c = p.c + c_off;
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int NP = kend > kbeg ? (kend - kbeg) / 64 : 0;  // pairs of k-tiles
    const int KT = 2 * NP;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

    typename Step::PlanA pa;
    typename Step::PlanB pb;
    pa.init(p.a_sm, p.a_sk, m0, p.M);
    pb.init(p.b_sn, p.b_sk, n0, p.N);
    const char* ta = p.a + a_off * 2 + Step::PlanA::origin(p.a_sm, p.a_sk, m0, kbeg);
    const char* tb = p.b + b_off * 2 + Step::PlanB::origin(p.b_sn, p.b_sk, n0, kbeg);
    const long long a_step = Step::PlanA::kstep(p.a_sk), b_step = Step::PlanB::kstep(p.b_sk);
    lds_char* const lds = (lds_char*)smem;
    lds_char* const ab = lds;                        // A pair slots
    lds_char* const bb = lds + A_SLOTS * A_SLOT;     // B slots
    asm volatile("" ::"s"(c), "s"(p.M), "s"(p.N));

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if (NP > 0) {
        // Prologue: virtual k-tiles -4 .. -1, each an A half then a B k-tile
        // (A pairs 0 and 1, B k-tiles 0 .. 2). ta / tb address the next pair
        // or k-tile to load, clamped to the last.
        {
            const char* ua = DmaPlan<BM, true, Step::NW, 64>::uniform(ta);
#pragma unroll
            for (int d = 0; d < PA; ++d) pa.issue_one(ab, ua, d);
#pragma unroll
            for (int d = 0; d < PA; ++d) pa.issue_one(ab, ua, PA + d);
            const char* ub = DmaPlan<BN, B_KC, Step::NW, 32>::uniform(tb);
            pb.issue(bb, ub);
            if (1 < NP) ta += a_step;
            if (1 < KT) tb += b_step;
            ua = DmaPlan<BM, true, Step::NW, 64>::uniform(ta);
#pragma unroll
            for (int d = 0; d < PA; ++d) pa.issue_one(ab + A_SLOT, ua, d);
            ub = DmaPlan<BN, B_KC, Step::NW, 32>::uniform(tb);
            pb.issue(bb + B_SLOT, ub);
            if (2 < KT) tb += b_step;
#pragma unroll
            for (int d = 0; d < PA; ++d) pa.issue_one(ab + A_SLOT, ua, PA + d);
            ub = DmaPlan<BN, B_KC, Step::NW, 32>::uniform(tb);
            pb.issue(bb + 2 * B_SLOT, ub);
            if (2 < NP) ta += a_step;
            if (3 < KT) tb += b_step;
        }
        // k-tile 0 (A pair 0, B k-tile 0) landed: loads of virtual k-tiles -2
        // and -1 may stay in flight.
        wait_vmcnt<4 * PA>();
        lds_barrier();
        u32x4_t fa[2][TM], fb[2][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[0][i] = frag<BM, true, 64>(ab, wm * WTM + i * 32, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[0][j] = frag<BN, B_KC, 32>(bb, wn * WTN + j * 32, 0);

        int aslot = 0, bslot = 0;
        constexpr int V = 3 * PA;  // loads of k-tile kt-1 and step 0 of kt
        for (int q = 0; q < NP; ++q) {
            const int aload = aslot == 0 ? 2 : aslot - 1;  // slot of pair q+2 (pair q-1's)
            const int anext = aslot == 2 ? 0 : aslot + 1;
            const lds_char* ra = ab + aslot * A_SLOT;
            lds_char* la = ab + aload * A_SLOT;
            const char* ua = DmaPlan<BM, true, Step::NW, 64>::uniform(ta);
            // ---- k-tile 2q (A half 0 of pair q+2)
            {
                const int bn = (bslot + 1) & 3, bl = (bslot + 3) & 3;
                const char* ub = DmaPlan<BN, B_KC, Step::NW, 32>::uniform(tb);
                Step::template run<0, 0>(acc, fa[0], fb[0], fa[1], fb[1], ra, 1, bb + bslot * B_SLOT, 1, wm, wn, la,
                                         bb + bl * B_SLOT, ua, ub, pa, pb);
                __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | (7 << 4));
                lds_barrier();
                Step::template run<1, 0>(acc, fa[1], fb[1], fa[0], fb[0], ra, 2, bb + bn * B_SLOT, 0, wm, wn, la,
                                         bb + bl * B_SLOT, ua, ub, pa, pb);
                if (2 * q + 4 < KT) tb += b_step;
                bslot = bn;
            }
            // ---- k-tile 2q+1 (A half 1 of pair q+2); the next k-tile reads pair q+1
            {
                const int bn = (bslot + 1) & 3, bl = (bslot + 3) & 3;
                const char* ub = DmaPlan<BN, B_KC, Step::NW, 32>::uniform(tb);
                Step::template run<0, 1>(acc, fa[0], fb[0], fa[1], fb[1], ra, 3, bb + bslot * B_SLOT, 1, wm, wn, la,
                                         bb + bl * B_SLOT, ua, ub, pa, pb);
                __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | (7 << 4));
                lds_barrier();
                Step::template run<1, 1>(acc, fa[1], fb[1], fa[0], fb[0], ab + anext * A_SLOT, 0, bb + bn * B_SLOT, 0,
                                         wm, wn, la, bb + bl * B_SLOT, ua, ub, pa, pb);
                if (2 * q + 5 < KT) tb += b_step;
                bslot = bn;
            }
            if (q + 3 < NP) ta += a_step;
            aslot = anext;
        }
        // No load may still be writing this workgroup's LDS when it exits.
        wait_vmcnt<0>();
    }

#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < p.M && col < p.N) c[(long long)row * p.N + col] = acc[i][j][r];
            }
        }
    }
}

// Direct-load 16-bit configurations (ORMI_GEMM_DMA_CFG):
//   two-stage, BK 64:  0: 256x256, 2x2 waves   1: 256x256, 2x4   2: 256x256, 4x2   3: 128x128, 2x2
//   multi-stage, BK 32: 4: 256x256, 2x2, 4 stages   5: 256x256, 2x4, 4 stages
//                       6: 256x256, 2x2, 5 stages   7: 256x256, 4x2, 4 stages
//   interleaved, BK 32: 8: 256x256, 2x2, 3 stages   9: 256x256, 2x2, 4 stages
//                       10: 256x256, 2x4, 4 stages  11: 256x256, 4x2, 4 stages
//   interleaved with whole-line A loads (A k-contiguous, K % 64 == 0, else 9):
//                       12: 256x256, 2x2, 3 A pair slots + 4 B slots
//   interleaved, BK 32, smaller tiles: 13: 128x128, 2x2, 4 stages (64 KB)
//                       14: 128x256, 2x2, 4 stages
//   whole-line A loads, 128x128: 15 (3 A pair slots + 4 B slots, 80 KB)
// The defaults: 15 (or 13) when 256x256 tiles do not fill the compute units;
// otherwise 12 where it applies (NN 4096^3 116.8 -> 112.4 us, NT 121.6 ->
// 114.3 us on one box, bit-identical), else 9, the fastest of 0-11 on MI355X
// for NN, NT and TN at 4096^3.
template <typename Tr, int BM, int BN, int WGM, int WGN>
struct DmaLauncher {
    static constexpr Cfg cfg{BM, BN, 64};
    template <bool A_KC, bool B_KC>
    static void go(const GemmParams& p, dim3 grid) {
        gemm_dma_kernel<Tr, BM, BN, WGM, WGN, A_KC, B_KC><<<grid, 64 * WGM * WGN>>>(p);
    }
    static void run(const GemmParams& p, dim3 grid, bool a_kc, bool b_kc) {
        if (a_kc && b_kc) go<true, true>(p, grid);
        else if (a_kc) go<true, false>(p, grid);
        else if (b_kc) go<false, true>(p, grid);
        else go<false, false>(p, grid);
    }
};
template <typename Tr, int BM, int BN, int BK, int WGM, int WGN, int STAGES>
struct PipeLauncher {
    static constexpr Cfg cfg{BM, BN, BK};
    template <bool A_KC, bool B_KC>
    static void go(const GemmParams& p, dim3 grid) {
        gemm_pipe_kernel<Tr, BM, BN, BK, WGM, WGN, STAGES, A_KC, B_KC><<<grid, 64 * WGM * WGN>>>(p);
    }
    static void run(const GemmParams& p, dim3 grid, bool a_kc, bool b_kc) {
        if (a_kc && b_kc) go<true, true>(p, grid);
        else if (a_kc) go<true, false>(p, grid);
        else if (b_kc) go<false, true>(p, grid);
        else go<false, false>(p, grid);
    }
};
template <typename Tr, int BM, int BN, int WGM, int WGN, int STAGES>
struct IlLauncher {
    static constexpr Cfg cfg{BM, BN, 32};
    template <bool A_KC, bool B_KC>
    static void go(const GemmParams& p, dim3 grid) {
        gemm_il_kernel<Tr, BM, BN, WGM, WGN, STAGES, A_KC, B_KC><<<grid, 64 * WGM * WGN>>>(p);
    }
    static void run(const GemmParams& p, dim3 grid, bool a_kc, bool b_kc) {
        if (a_kc && b_kc) go<true, true>(p, grid);
        else if (a_kc) go<true, false>(p, grid);
        else if (b_kc) go<false, true>(p, grid);
        else go<false, false>(p, grid);
    }
};
// Whole-line A loads (gemm_ilp_kernel) for a k-contiguous A; the interleaved
// 4-stage kernel otherwise.
template <typename Tr, int BM, int BN, int WGM, int WGN>
struct IlpLauncher {
    static constexpr Cfg cfg{BM, BN, 64};
    static void run(const GemmParams& p, dim3 grid, bool a_kc, bool b_kc) {
        if (a_kc && b_kc) gemm_ilp_kernel<Tr, BM, BN, WGM, WGN, true><<<grid, 64 * WGM * WGN>>>(p);
        else if (a_kc) gemm_ilp_kernel<Tr, BM, BN, WGM, WGN, false><<<grid, 64 * WGM * WGN>>>(p);
        else IlLauncher<Tr, BM, BN, WGM, WGN, 4>::run(p, grid, a_kc, b_kc);
    }
};
template <typename Tr>
static Cfg cfg_dma(int id) {
    switch (id) {
        case 0: return DmaLauncher<Tr, 256, 256, 2, 2>::cfg;
        case 1: return DmaLauncher<Tr, 256, 256, 2, 4>::cfg;
        case 2: return DmaLauncher<Tr, 256, 256, 4, 2>::cfg;
        case 3: return DmaLauncher<Tr, 128, 128, 2, 2>::cfg;
        case 4: return PipeLauncher<Tr, 256, 256, 32, 2, 2, 4>::cfg;
        case 5: return PipeLauncher<Tr, 256, 256, 32, 2, 4, 4>::cfg;
        case 6: return PipeLauncher<Tr, 256, 256, 32, 2, 2, 5>::cfg;
        case 7: return PipeLauncher<Tr, 256, 256, 32, 4, 2, 4>::cfg;
        case 8: return IlLauncher<Tr, 256, 256, 2, 2, 3>::cfg;
        case 9: return IlLauncher<Tr, 256, 256, 2, 2, 4>::cfg;
        case 10: return IlLauncher<Tr, 256, 256, 2, 4, 4>::cfg;
        case 12: return IlpLauncher<Tr, 256, 256, 2, 2>::cfg;
        case 13: return IlLauncher<Tr, 128, 128, 2, 2, 4>::cfg;
        case 14: return IlLauncher<Tr, 128, 256, 2, 2, 4>::cfg;
        case 15: return IlpLauncher<Tr, 128, 128, 2, 2>::cfg;
        default: return IlLauncher<Tr, 256, 256, 4, 2, 4>::cfg;
    }
}
template <typename Tr>
static void run_dma(int id, const GemmParams& p, dim3 grid, bool a_kc, bool b_kc) {
    switch (id) {
        case 0: DmaLauncher<Tr, 256, 256, 2, 2>::run(p, grid, a_kc, b_kc); break;
        case 1: DmaLauncher<Tr, 256, 256, 2, 4>::run(p, grid, a_kc, b_kc); break;
        case 2: DmaLauncher<Tr, 256, 256, 4, 2>::run(p, grid, a_kc, b_kc); break;
        case 3: DmaLauncher<Tr, 128, 128, 2, 2>::run(p, grid, a_kc, b_kc); break;
        case 4: PipeLauncher<Tr, 256, 256, 32, 2, 2, 4>::run(p, grid, a_kc, b_kc); break;
        case 5: PipeLauncher<Tr, 256, 256, 32, 2, 4, 4>::run(p, grid, a_kc, b_kc); break;
        case 6: PipeLauncher<Tr, 256, 256, 32, 2, 2, 5>::run(p, grid, a_kc, b_kc); break;
        case 7: PipeLauncher<Tr, 256, 256, 32, 4, 2, 4>::run(p, grid, a_kc, b_kc); break;
        case 8: IlLauncher<Tr, 256, 256, 2, 2, 3>::run(p, grid, a_kc, b_kc); break;
        case 9: IlLauncher<Tr, 256, 256, 2, 2, 4>::run(p, grid, a_kc, b_kc); break;
        case 10: IlLauncher<Tr, 256, 256, 2, 4, 4>::run(p, grid, a_kc, b_kc); break;
        case 12: IlpLauncher<Tr, 256, 256, 2, 2>::run(p, grid, a_kc, b_kc); break;
        case 13: IlLauncher<Tr, 128, 128, 2, 2, 4>::run(p, grid, a_kc, b_kc); break;
        case 14: IlLauncher<Tr, 128, 256, 2, 2, 4>::run(p, grid, a_kc, b_kc); break;
        case 15: IlpLauncher<Tr, 128, 128, 2, 2>::run(p, grid, a_kc, b_kc); break;
        default: IlLauncher<Tr, 256, 256, 4, 2, 4>::run(p, grid, a_kc, b_kc); break;
    }
}

// Split-K workspace, grown on demand and kept; every use is ordered on the
// null stream, so reuse by the next call is safe. g_ws_mu is held from the
// moment a call takes the workspace until its kernels are enqueued, so another
// host thread can neither free it nor interleave its own launches that use it.
static std::mutex g_ws_mu;
static void* g_ws = nullptr;
static size_t g_ws_bytes = 0;

// Caller holds g_ws_mu.
static int workspace_locked(size_t bytes, void** out) {
    if (bytes > g_ws_bytes) {
        if (g_ws) {
            hipError_t e = hipDeviceSynchronize();
            if (e == hipSuccess) e = hipFree(g_ws);
            if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("gemm workspace free: ") + hipGetErrorString(e));
            g_ws = nullptr;
            g_ws_bytes = 0;
        }
        hipError_t e = hipMalloc(&g_ws, bytes);
        if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("gemm workspace: ") + hipGetErrorString(e));
        g_ws_bytes = bytes;
    }
    *out = g_ws;
    return ORMI_HIP_OK;
}

// Workspace of the allocation-free entry (ormi_hip_gemm_ex_noalloc): split-K
// partials and the input of the finish pass live in this array, which the
// code object carries, so no call allocates. The device holds it for the life
// of the process. In host code `scratch` names a host-side stand-in, not device
// memory: kernels and copies get g_scratch, its device address, which
// gemm_scratch_setup resolves once, with the bound device current. Every call
// reuses the same bytes (a call's kernels overwrite everything the next one
// reads: each split's kernel stores its whole partial slice).
static __device__ __align__(256) unsigned char scratch[ORMI_GEMM_NOALLOC_SCRATCH_BYTES];
static void* g_scratch = nullptr;

static int scratch_locked(size_t bytes, void** out) {
    if (bytes > ORMI_GEMM_NOALLOC_SCRATCH_BYTES)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm_ex_noalloc: this shape needs " + std::to_string(bytes) +
                                              " bytes of workspace; the allocation-free entry holds at most " +
                                              std::to_string((size_t)ORMI_GEMM_NOALLOC_SCRATCH_BYTES) +
                                              " (use ormi_hip_gemm_ex)");
    if (!g_scratch) return fail(ORMI_HIP_ERR_RUNTIME, "ormi_hip_gemm_ex_noalloc: scratch address not resolved");
    *out = g_scratch;
    return ORMI_HIP_OK;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int gemm_scratch_setup() {
    const hipError_t e = hipGetSymbolAddress(&g_scratch, HIP_SYMBOL(scratch));
    if (e != hipSuccess) {
        g_scratch = nullptr;
        return fail(ORMI_HIP_ERR_RUNTIME, std::string("gemm scratch: hipGetSymbolAddress: ") + hipGetErrorString(e));
    }
    return ORMI_HIP_OK;
}

}  // namespace ormi_hip

using namespace ormi_hip;

namespace ormi_hip {
// Element offsets [lo, hi] an operand with these extents and strides spans.
static void span(long long ext, long long stride, long long* lo, long long* hi) {
    if (ext <= 1 || stride == 0) return;
    const long long reach = (ext - 1) * stride;
    if (reach < 0) *lo += reach;
    else *hi += reach;
}

// The epilogue as the kernels take it; an error for a malformed one.
static int make_epi(const ormi_gemm_desc* d, const ormi_gemm_epilogue* in, long long batch, Epi* out) {
    *out = Epi{};
    out->kind = ORMI_GEMM_EPI_NONE;
    if (!in || in->kind == ORMI_GEMM_EPI_NONE) return ORMI_HIP_OK;
    if (in->kind < ORMI_GEMM_EPI_ADD || in->kind > ORMI_GEMM_EPI_MUL_FN_D)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm_ex: unknown epilogue kind");
    if (in->fn < ORMI_GEMM_FN_IDENTITY || in->fn > ORMI_GEMM_FN_GELU_GRAD)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm_ex: unknown epilogue function");
    if (in->kind == ORMI_GEMM_EPI_ADD && (in->form < 0 || in->form > 2))
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm_ex: ADD form must be 0, 1 or 2");
    const bool needs_d = in->kind == ORMI_GEMM_EPI_ADD || in->kind == ORMI_GEMM_EPI_MUL_FN_D;
    if (needs_d && !in->d) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm_ex: epilogue needs D");
    auto misaligned = [](const void* q) { return ((uintptr_t)q & 3u) != 0; };
    if ((needs_d && misaligned(in->d)) || (in->s && misaligned(in->s)) || (in->aux && misaligned(in->aux)))
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm_ex: epilogue operands must be 4-byte aligned");
    const float* c0 = d->c;
    const float* c1 = d->c + batch * d->M * d->N;
    const bool aux_used = in->kind == ORMI_GEMM_EPI_UNARY && in->aux;
    if (aux_used && in->aux < c1 && in->aux + batch * d->M * d->N > c0)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm_ex: aux overlaps C");
    long long d_lo = 0, d_hi = 0;
    if (needs_d) {
        span(d->M, in->d_stride_m, &d_lo, &d_hi);
        span(d->N, in->d_stride_n, &d_lo, &d_hi);
        for (int i = 0; i < d->batch_ndim; ++i) span(d->batch_shape[i], in->d_batch_stride[i], &d_lo, &d_hi);
    }
    const intptr_t dp = (intptr_t)in->d, cb = (intptr_t)c0, ce = (intptr_t)c1;
    if (needs_d && dp + d_lo * 4 < ce && dp + d_hi * 4 >= cb) {
        // D overlaps C anywhere in its span: allowed in place only, with C's own
        // layout, where each element is read before the same thread writes it.
        bool same = in->d == c0 && in->d_stride_m == d->N && in->d_stride_n == 1;
        long long contig = (long long)d->M * d->N;
        for (int i = d->batch_ndim - 1; i >= 0 && same; --i) {
            same = in->d_batch_stride[i] == contig || d->batch_shape[i] == 1;
            contig *= d->batch_shape[i];
        }
        if (!same) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm_ex: D overlaps C with another layout");
    }
    out->kind = in->kind;
    out->fn = in->fn;
    out->form = in->form;
    out->s = in->kind == ORMI_GEMM_EPI_ADD ? in->s : nullptr;
    out->d = needs_d ? in->d : nullptr;
    out->d_sm = needs_d ? in->d_stride_m : 0;
    out->d_sn = needs_d ? in->d_stride_n : 0;
    for (int i = 0; i < ORMI_GEMM_MAX_BATCH_DIMS; ++i) out->d_bs[i] = needs_d && i < d->batch_ndim ? in->d_batch_stride[i] : 0;
    out->aux = aux_used ? in->aux : nullptr;
    return ORMI_HIP_OK;
}

static void launch_finish(const ormi_gemm_desc* d, const float* ws, int splits, long long batch, const Epi& epi) {
    FinishParams f{};
    f.c = d->c;
    f.ws = ws;
    f.n = batch * d->M * d->N;
    f.splits = splits;
    f.M = d->M;
    f.N = d->N;
    f.rows = (int)(batch * d->M);
    f.batch_ndim = d->batch_ndim;
    for (int i = 0; i < d->batch_ndim; ++i) f.batch_shape[i] = d->batch_shape[i];
    f.epi = epi;
    const bool vec = d->N % 4 == 0 && ((uintptr_t)d->c & 15u) == 0 && ((uintptr_t)epi.aux & 15u) == 0;
    if (vec && epi.kind == ORMI_GEMM_EPI_NONE) {
        constexpr int U = 4;
        const long long n4 = f.n / 4;
        const long long blocks = std::max(1LL, std::min((n4 + 256LL * U - 1) / (256LL * U), (long long)compute_units() * 8));
        gemm_finish_flat_kernel<U><<<(unsigned)blocks, 256>>>(f.c, ws, n4, splits);
        return;
    }
    const int gx = std::min((d->N + 1023) / 1024, 64);
    const int gy = std::max(1, std::min({f.rows, compute_units() * 32 / gx, 65535}));
    if (vec) gemm_finish_kernel<true><<<dim3(gx, gy), 256>>>(f);
    else gemm_finish_kernel<false><<<dim3(gx, gy), 256>>>(f);
}
}  // namespace ormi_hip

namespace ormi_hip {
// Both GEMM entries: noalloc takes the workspace from `scratch` instead of the
// grown-on-demand buffer.
static int gemm_run_locked(const ormi_gemm_desc* d, const Epi& epi, long long batch, bool noalloc, bool packed);
static int gemm_packed_locked(const ormi_gemm_desc* d, const Epi& epi, long long batch);

// Checks one call's arguments and converts its epilogue; *nothing is set when
// the product has no elements (nothing to launch).
static int gemm_check(const ormi_gemm_desc* d, const ormi_gemm_epilogue* epi_in, long long* batch_out, Epi* epi,
                      bool* nothing) {
    *nothing = false;
    if (!d) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: null descriptor");
    if (d->M < 0 || d->N < 0 || d->K < 0) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: negative dimension");
    if (d->batch_ndim < 0 || d->batch_ndim > ORMI_GEMM_MAX_BATCH_DIMS)
        return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: batch_ndim must be 0..4");
    if (d->dtype != ORMI_DTYPE_F32 && d->dtype != ORMI_DTYPE_BF16 && d->dtype != ORMI_DTYPE_F16)
        return fail(ORMI_HIP_ERR_UNSUPPORTED, "ormi_hip_gemm: dtype must be f32, bf16 or f16");
    long long batch = 1;
    for (int i = 0; i < d->batch_ndim; ++i) {
        if (d->batch_shape[i] <= 0) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: batch extents must be positive");
        batch *= d->batch_shape[i];  // <= 65535 * (2^31 - 1) before the check below: no overflow
        if (batch > 65535) return fail(ORMI_HIP_ERR_UNSUPPORTED, "ormi_hip_gemm: more than 65535 batches");
    }
    *batch_out = batch;
    if ((long long)d->M * d->N == 0) {
        *nothing = true;
        return ORMI_HIP_OK;
    }
    // With K == 0 the operands hold no elements (an empty buffer may have no
    // address) and are never read.
    if (!d->c || (d->K > 0 && (!d->a || !d->b))) return fail(ORMI_HIP_ERR_INVALID, "ormi_hip_gemm: null operand");
    if (batch * d->M > 0x7fffffffLL) return fail(ORMI_HIP_ERR_UNSUPPORTED, "ormi_hip_gemm: more than 2^31 output rows");
    return make_epi(d, epi_in, batch, epi);
}

static int gemm_run(const ormi_gemm_desc* d, const ormi_gemm_epilogue* epi_in, bool noalloc) {
    long long batch = 1;
    Epi epi;
    bool nothing = false;
    int rc = gemm_check(d, epi_in, &batch, &epi, &nothing);
    if (rc != ORMI_HIP_OK || nothing) return rc;
    rc = ensure_init();
    if (rc != ORMI_HIP_OK) return rc;
    rc = drain_queue();
    if (rc != ORMI_HIP_OK) return rc;

    // Held until this call's kernels are enqueued (see g_ws_mu).
    std::lock_guard<std::mutex> ws_lock(g_ws_mu);
    return gemm_run_locked(d, epi, batch, noalloc, false);
}

// ------------------------------------------------------------ GEMM pairs --
// Whether product d (one batch) runs alone as fp32 direct-load configuration
// 1 with whole 128x128 tiles, no K split and its epilogue in the store: the
// conditions gemm_run_locked takes that path under, so that the pair kernel,
// which computes each tile as that path does, gives the same bits. a_kc /
// b_kc: the operand layouts that path would use.
static bool pair_eligible(const ormi_gemm_desc* d, const Epi& epi, long long batch, bool* a_kc, bool* b_kc) {
    if (d->dtype != ORMI_DTYPE_F32 || batch != 1 || d->K <= 0) return false;
    if (env_cfg("ORMI_GEMM_F32_DMA", 1) == 0) return false;
    *a_kc = d->a_stride_k == 1;
    *b_kc = d->b_stride_k == 1;
    const bool a_mc = d->a_stride_m == 1, b_nc = d->b_stride_n == 1;
    if (!(*a_kc || a_mc) || !(*b_kc || b_nc) || !aligned16(d->a) || !aligned16(d->b)) return false;
    const long long a_other = *a_kc ? d->a_stride_m : d->a_stride_k;
    const long long b_other = *b_kc ? d->b_stride_n : d->b_stride_k;
    if (a_other % 4 != 0 || b_other % 4 != 0) return false;
    if (d->M % 128 != 0 || d->N % 128 != 0 || d->K % 32 != 0) return false;  // whole tiles (and 16-byte chunks)
    const long long a_span32 = *a_kc ? 256LL * d->a_stride_m * 4 : 64LL * d->a_stride_k * 4 + 1024;
    const long long b_span32 = *b_kc ? 256LL * d->b_stride_n * 4 : 64LL * d->b_stride_k * 4 + 1024;
    if (a_span32 >= (1LL << 32) || b_span32 >= (1LL << 32)) return false;
    // Configuration 1 without a K split: at least one tile per compute unit.
    const long long tiles = (long long)(d->M / 128) * (d->N / 128);
    const int forced = env_cfg("ORMI_GEMM_F32_DMA_CFG", -1);
    if ((forced >= 0 && forced <= 9 && forced != 1) || tiles < compute_units()) return false;
    return epi.kind == ORMI_GEMM_EPI_NONE || (epi.kind != ORMI_GEMM_EPI_UNARY && epi_in_store(epi));
}

// Byte ranges [lo, hi) a product reads and writes (one batch).
struct Ranges {
    intptr_t r_lo[4], r_hi[4], w_lo[2], w_hi[2];
    int nr = 0, nw = 0;
};
static void add_range(intptr_t* lo, intptr_t* hi, int* n, const void* base, long long e_lo, long long e_hi) {
    lo[*n] = (intptr_t)base + (intptr_t)e_lo * 4;
    hi[*n] = (intptr_t)base + (intptr_t)e_hi * 4 + 4;
    ++*n;
}
static Ranges ranges_of(const ormi_gemm_desc* d, const Epi& epi) {
    Ranges r;
    long long lo = 0, hi = 0;
    span(d->M, d->a_stride_m, &lo, &hi);
    span(d->K, d->a_stride_k, &lo, &hi);
    add_range(r.r_lo, r.r_hi, &r.nr, d->a, lo, hi);
    lo = hi = 0;
    span(d->K, d->b_stride_k, &lo, &hi);
    span(d->N, d->b_stride_n, &lo, &hi);
    add_range(r.r_lo, r.r_hi, &r.nr, d->b, lo, hi);
    if (epi_reads_d(epi)) {
        lo = hi = 0;
        span(d->M, epi.d_sm, &lo, &hi);
        span(d->N, epi.d_sn, &lo, &hi);
        add_range(r.r_lo, r.r_hi, &r.nr, epi.d, lo, hi);
    }
    if (epi.kind != ORMI_GEMM_EPI_NONE && epi.s) add_range(r.r_lo, r.r_hi, &r.nr, epi.s, 0, 0);
    const long long mn = (long long)d->M * d->N;
    add_range(r.w_lo, r.w_hi, &r.nw, d->c, 0, mn - 1);
    if (epi.kind == ORMI_GEMM_EPI_UNARY && epi.aux) add_range(r.w_lo, r.w_hi, &r.nw, epi.aux, 0, mn - 1);
    return r;
}
// Whether running x and y in either order (or at once) gives the same result:
// neither writes what the other reads or writes.
static bool independent(const Ranges& x, const Ranges& y) {
    auto meet = [](intptr_t a0, intptr_t a1, intptr_t b0, intptr_t b1) { return a0 < b1 && b0 < a1; };
    for (int i = 0; i < x.nw; ++i) {
        for (int j = 0; j < y.nr; ++j)
            if (meet(x.w_lo[i], x.w_hi[i], y.r_lo[j], y.r_hi[j])) return false;
        for (int j = 0; j < y.nw; ++j)
            if (meet(x.w_lo[i], x.w_hi[i], y.w_lo[j], y.w_hi[j])) return false;
    }
    for (int i = 0; i < y.nw; ++i)
        for (int j = 0; j < x.nr; ++j)
            if (meet(y.w_lo[i], y.w_hi[i], x.r_lo[j], x.r_hi[j])) return false;
    return true;
}

static GemmParams pair_params(const ormi_gemm_desc* d, const Epi& epi) {
    GemmParams p{};
    p.a = (const char*)d->a;
    p.b = (const char*)d->b;
    p.c = d->c;
    p.M = d->M; p.N = d->N; p.K = d->K;
    p.a_sm = d->a_stride_m; p.a_sk = d->a_stride_k;
    p.b_sk = d->b_stride_k; p.b_sn = d->b_stride_n;
    p.batch = 1;
    p.splits = 1;
    p.k_per_split = d->K;
    p.tiles_m = d->M / 128;
    p.tiles_n = d->N / 128;
    p.epi = epi;
    return p;
}

static int gemm_pair(const ormi_gemm_desc* d0, const ormi_gemm_epilogue* e0, const ormi_gemm_desc* d1,
                     const ormi_gemm_epilogue* e1, int* grouped) {
    if (grouped) *grouped = 0;
    long long b0 = 1, b1 = 1;
    Epi epi0, epi1;
    bool none0 = false, none1 = false;
    int rc = gemm_check(d0, e0, &b0, &epi0, &none0);
    if (rc != ORMI_HIP_OK) return rc;
    rc = gemm_check(d1, e1, &b1, &epi1, &none1);
    if (rc != ORMI_HIP_OK) return rc;
    rc = ensure_init();
    if (rc != ORMI_HIP_OK) return rc;
    rc = drain_queue();
    if (rc != ORMI_HIP_OK) return rc;
    std::lock_guard<std::mutex> ws_lock(g_ws_mu);
    bool ak0 = false, bk0 = false, ak1 = false, bk1 = false;
    const int mode = env_cfg("ORMI_GEMM_PAIR", 1);
    if (!none0 && !none1 && mode != 0 && pair_eligible(d0, epi0, b0, &ak0, &bk0) &&
        pair_eligible(d1, epi1, b1, &ak1, &bk1) && independent(ranges_of(d0, epi0), ranges_of(d1, epi1))) {
        const GemmParams p0 = pair_params(d0, epi0), p1 = pair_params(d1, epi1);
        const long long t0 = (long long)p0.tiles_m * p0.tiles_n, t1 = (long long)p1.tiles_m * p1.tiles_n;
        const int groups = (int)std::min<long long>(compute_units(), t0 + t1);
        // Grouping pays while each work-group's stream is short: one box, dX
        // (1024 x 4096, TT, gelu') with dW (4096 x 1024, FF, SGD), both at
        // depth K, two launches -> one: K 64 28.0 -> 26.4 us, 256 50.6 ->
        // 48.4, 512 79.1 -> 76.0, 1024 (64 k-tiles per work-group) 136.9 ->
        // 134.2; C5's layer-2 pair (256 k-tiles per work-group) 499.8 -> 501.3.
        // So by default (1) only streams of at most kPairMaxKTiles k-tiles per
        // work-group are grouped; 2 groups every eligible pair.
        constexpr long long kPairMaxKTiles = 64;
        const long long per_group = (t0 * (p0.K / 32) + t1 * (p1.K / 32) + groups - 1) / groups;
        // The kernel takes the products in one order of layouts; independent
        // products may run in either.
        const bool launched = (mode == 2 || per_group <= kPairMaxKTiles) &&
                              (run32_dma_pair(p0, ak0, bk0, p1, ak1, bk1, groups) ||
                               run32_dma_pair(p1, ak1, bk1, p0, ak0, bk0, groups));
        if (launched) {
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("ormi_hip_gemm_pair launch: ") + hipGetErrorString(e));
            if (grouped) *grouped = 1;
            return ORMI_HIP_OK;
        }
    }
    // Otherwise the two products in order, each as its own call would run.
    if (!none0) rc = gemm_run_locked(d0, epi0, b0, false, false);
    if (rc != ORMI_HIP_OK || none1) return rc;
    return gemm_run_locked(d1, epi1, b1, false, false);
}

// Packed operands (gemm_pack_kernel), grown on demand and kept, like the
// split-K workspace; used under g_ws_mu.
static void* g_pack = nullptr;
static size_t g_pack_bytes = 0;

static int gemm_packed_locked(const ormi_gemm_desc* d, const Epi& epi, long long batch) {
    const int es = d->dtype == ORMI_DTYPE_F32 ? 4 : 2;
    const int k_pad = (int)(((long long)d->K + 63) / 64 * 64);
    if (k_pad < d->K) return fail(ORMI_HIP_ERR_UNSUPPORTED, "ormi_hip_gemm: K too large to pack");
    auto round256 = [](size_t v) { return (v + 255) / 256 * 256; };
    const size_t a_bytes = round256((size_t)batch * d->M * k_pad * es);
    const size_t b_bytes = round256((size_t)batch * d->N * k_pad * es);
    if (a_bytes + b_bytes > g_pack_bytes) {
        if (g_pack) {
            hipError_t e = hipDeviceSynchronize();
            if (e == hipSuccess) e = hipFree(g_pack);
            if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("gemm pack buffer free: ") + hipGetErrorString(e));
            g_pack = nullptr;
            g_pack_bytes = 0;
        }
        const hipError_t e = hipMalloc(&g_pack, a_bytes + b_bytes);
        if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("gemm pack buffer: ") + hipGetErrorString(e));
        g_pack_bytes = a_bytes + b_bytes;
    }
    char* const pa = (char*)g_pack;
    char* const pb = pa + a_bytes;
    auto pack = [&](void* dst, const void* src, int mn, long long s_mn, long long s_k, const int64_t* bs) {
        PackParams pp{};
        pp.s_mn = s_mn;
        pp.s_k = s_k;
        pp.MN = mn;
        pp.K = d->K;
        pp.K_pad = k_pad;
        pp.batch_ndim = d->batch_ndim;
        for (int i = 0; i < d->batch_ndim; ++i) {
            pp.batch_shape[i] = d->batch_shape[i];
            pp.bs[i] = bs[i];
        }
        const dim3 grid(k_pad / 64, (mn + 63) / 64, (unsigned)batch);
        const bool mn_unit = s_mn == 1 && s_k != 1;
        if (es == 4) {
            if (mn_unit) gemm_pack_kernel<float, true><<<grid, 256>>>((float*)dst, (const float*)src, pp);
            else gemm_pack_kernel<float, false><<<grid, 256>>>((float*)dst, (const float*)src, pp);
        } else {
            if (mn_unit) gemm_pack_kernel<unsigned short, true><<<grid, 256>>>((unsigned short*)dst, (const unsigned short*)src, pp);
            else gemm_pack_kernel<unsigned short, false><<<grid, 256>>>((unsigned short*)dst, (const unsigned short*)src, pp);
        }
    };
    pack(pa, d->a, d->M, d->a_stride_m, d->a_stride_k, d->a_batch_stride);
    pack(pb, d->b, d->N, d->b_stride_n, d->b_stride_k, d->b_batch_stride);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("ormi_hip_gemm pack: ") + hipGetErrorString(e));
    // The packed product: both operands k-contiguous over K_pad, dense batches.
    ormi_gemm_desc dp = *d;
    dp.K = k_pad;
    dp.a = pa;
    dp.a_stride_m = k_pad;
    dp.a_stride_k = 1;
    dp.b = pb;
    dp.b_stride_n = k_pad;
    dp.b_stride_k = 1;
    long long inner = 1;
    for (int i = d->batch_ndim - 1; i >= 0; --i) {
        dp.a_batch_stride[i] = inner * d->M * k_pad;
        dp.b_batch_stride[i] = inner * d->N * k_pad;
        inner *= d->batch_shape[i];
    }
    return gemm_run_locked(&dp, epi, batch, false, true);
}

static int gemm_run_locked(const ormi_gemm_desc* d, const Epi& epi, long long batch, bool noalloc, bool packed) {
    int rc = ORMI_HIP_OK;
    auto workspace = [noalloc](size_t bytes, void** out) {
        return noalloc ? scratch_locked(bytes, out) : workspace_locked(bytes, out);
    };

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
    p.batch = (int)batch;
    p.splits = 1;
    p.k_per_split = d->K;
    p.epi = epi;

    if (d->K == 0) {
        // The product is 0; with an epilogue, 0 goes through it.
        const float zero = 0.0f;
        const size_t out_elems = (size_t)batch * d->M * d->N;
        if (epi.kind == ORMI_GEMM_EPI_NONE) return ormi_hip_fill(d->c, &zero, 4, out_elems);
        void* ws = nullptr;
        rc = workspace(out_elems * sizeof(float), &ws);
        if (rc == ORMI_HIP_OK) rc = ormi_hip_fill(ws, &zero, 4, out_elems);
        if (rc != ORMI_HIP_OK) return rc;
        launch_finish(d, (const float*)ws, 1, batch, epi);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("ormi_hip_gemm launch: ") + hipGetErrorString(e));
        return ORMI_HIP_OK;
    }

    const bool f32 = d->dtype == ORMI_DTYPE_F32;
    const int VE = f32 ? 4 : 8;
    // Which index is unit-stride for each operand (k preferred when both are).
    const bool a_kc = d->a_stride_k == 1, a_mc = d->a_stride_m == 1;
    const bool b_kc = d->b_stride_k == 1, b_nc = d->b_stride_n == 1;
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

    hipError_t e;
    // Operands the fast kernels cannot take are packed into dense k-contiguous
    // buffers first, unless the product is small (the generic kernel is then
    // at its launch floor anyway) or the caller cannot allocate.
    if (!fast && !packed && !noalloc && (long long)d->M * d->N * d->K >= (1LL << 24) &&
        env_cfg("ORMI_GEMM_PACK", 1) != 0)
        return gemm_packed_locked(d, epi, batch);
    if (!fast) {
        dim3 grid((d->N + 15) / 16, (d->M + 15) / 16, (unsigned)batch);
        if (f32) gemm_generic_kernel<ORMI_DTYPE_F32><<<grid, 256>>>(p);
        else if (d->dtype == ORMI_DTYPE_BF16) gemm_generic_kernel<ORMI_DTYPE_BF16><<<grid, 256>>>(p);
        else gemm_generic_kernel<ORMI_DTYPE_F16><<<grid, 256>>>(p);
        e = hipGetLastError();
        if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("ormi_hip_gemm launch: ") + hipGetErrorString(e));
        return ORMI_HIP_OK;
    }

    // Direct-load path: 16-bit, K in whole tiles of the configuration's depth,
    // the mn-contiguous operand's extent in whole 16-byte chunks.
    // Per-lane load offsets within one tile are 32-bit: a tile (at most 256
    // rows of k-contiguous data, or 64 k-rows of mn-contiguous data) spans
    // less than 4 GB.
    const long long a_span = a_kc ? 256LL * d->a_stride_m * 2 : 64LL * d->a_stride_k * 2 + 512;
    const long long b_span = b_kc ? 256LL * d->b_stride_n * 2 : 64LL * d->b_stride_k * 2 + 512;
    // Default: 256x256 tiles when they alone fill the compute units, else
    // 128x128 tiles with two work-groups per compute unit (one box: 2048^2 x
    // 1024 35.4 -> 14.0 us, 3072^3 96.3 -> 66.7 us, 512 x 4096^2 37.8 -> 26.9
    // us); either with whole-line A loads (12, 15) if A is k-contiguous and K
    // is in whole 64-deep pairs, else the interleaved 4-stage kernel (9, 13).
    const long long tiles256 = (long long)((d->M + 255) / 256) * ((d->N + 255) / 256) * batch;
    const bool whole_line = a_kc && d->K % 64 == 0;
    const int dma_dflt = tiles256 < compute_units() ? (whole_line ? 15 : 13) : (whole_line ? 12 : 9);
    const int dma_id = env_cfg("ORMI_GEMM_DMA_CFG", dma_dflt);
    const int dma_bk = f32 ? 64 : cfg_dma<TrBF16>(dma_id).BK;
    const bool dma = !f32 && env_cfg("ORMI_GEMM_DMA", 1) != 0 && d->K % dma_bk == 0 && (a_kc || d->M % 8 == 0) &&
                     (b_kc || d->N % 8 == 0) && a_span < (1LL << 32) && b_span < (1LL << 32);
    // fp32 with direct loads: K in whole 32-deep tiles, mn-contiguous extents
    // in whole 16-byte chunks, per-lane tile offsets in 32 bits.
    const long long a_span32 = a_kc ? 256LL * d->a_stride_m * 4 : 64LL * d->a_stride_k * 4 + 1024;
    const long long b_span32 = b_kc ? 256LL * d->b_stride_n * 4 : 64LL * d->b_stride_k * 4 + 1024;
    // Default fp32 configuration: 128x128 tiles (1), or 128x64 tiles (9; 6
    // when K is not in whole 64-deep tiles) when 128x128 tiles would leave
    // compute units idle. Twice the tiles then need half the K split or none:
    // one box, interleaved, warm clocks: 2048x1024x4096 NT (C4's dA) 128.6 ->
    // 124.9 us, 1024^2 x 4096 NN 69.3 -> 67.9, 1024x2048x2048 TN 69.6 ->
    // 63.3, 2048x1024x1024 NT 40.3 -> 34.9, 512^2 x 4096 30.9 -> 26.9.
    int dma32_id = env_cfg("ORMI_GEMM_F32_DMA_CFG", -1);
    if (dma32_id < 0 || dma32_id > 9) {
        const long long t128 = (long long)((d->M + 127) / 128) * ((d->N + 127) / 128) * batch;
        dma32_id = t128 >= compute_units() ? 1 : d->K % 64 == 0 ? 9 : 6;
    }
    int dma32_bm = 0, dma32_bn = 0, dma32_bk = 0;
    cfg32_dma(dma32_id, &dma32_bm, &dma32_bn, &dma32_bk);
    const bool dma32 = f32 && env_cfg("ORMI_GEMM_F32_DMA", 1) != 0 && d->K % dma32_bk == 0 && (a_kc || d->M % 4 == 0) &&
                       (b_kc || d->N % 4 == 0) && a_span32 < (1LL << 32) && b_span32 < (1LL << 32);
    // A large product whose layout the direct-load kernels cannot take (K not
    // in whole tiles, an mn-contiguous extent not in whole 16-byte chunks) is
    // packed for them too, rather than run on the register-staged kernels: one
    // box, fp32 3000^2 x 1000 218.7 -> 203.5 us, 2000 x 4000 x 1000 161.5 ->
    // 153.8 us. Below 2^32 multiply-adds the packing costs more than it gains
    // (fp32 1000^3 33.7 -> 47.5 us).
    const bool direct_on = env_cfg(f32 ? "ORMI_GEMM_F32_DMA" : "ORMI_GEMM_DMA", 1) != 0;
    if (!packed && !noalloc && direct_on && !(f32 ? dma32 : dma) && (long long)d->M * d->N * d->K >= (1LL << 32) &&
        env_cfg("ORMI_GEMM_PACK", 1) != 0)
        return gemm_packed_locked(d, epi, batch);
    int id = dma ? dma_id
             : dma32 ? dma32_id
             : f32 ? env_cfg("ORMI_GEMM_CFG32", -1)
                   : env_cfg("ORMI_GEMM_CFG16", 0);
    if (f32 && !dma32 && id < 0) {
        // 128x256 tiles (config 2) for M and N in whole 128x256 tiles, unless
        // they cannot fill the compute units and K is short: then 128x128
        // tiles (config 3) fill them without a K split, whose partial round
        // trip and second kernel cost more than the smaller tiles lose at
        // K <= 1024 (measured: 1024x4096x1024 86 us against 94 us split; at
        // K = 2048 the split is 4% faster). Shapes with a partial tile take
        // config 3: config 2 measured 16-29% slower on 3000x3000x1000,
        // 2500x4000x1500, 4100x4100x512 and 5000^3, and config 3 18% faster
        // than either other on 3000x4096x1024, within 8% of the best on all.
        const long long cus_ll = compute_units();
        const long long t2 = (long long)((d->M + 127) / 128) * ((d->N + 255) / 256) * batch;
        const long long t3 = (long long)((d->M + 127) / 128) * ((d->N + 127) / 128) * batch;
        const bool whole2 = d->M % 128 == 0 && d->N % 256 == 0;
        id = (!whole2 || (t2 < cus_ll && t3 >= cus_ll && d->K <= 1024)) ? 3 : 2;
    }
    const Cfg cf = [&] {
        if (dma) return d->dtype == ORMI_DTYPE_BF16 ? cfg_dma<TrBF16>(id) : cfg_dma<TrF16>(id);
        if (dma32) return Cfg{dma32_bm, dma32_bn, dma32_bk};
        return f32 ? cfg32(id) : (d->dtype == ORMI_DTYPE_BF16 ? cfg16<TrBF16>(id) : cfg16<TrF16>(id));
    }();
    p.tiles_m = (d->M + cf.BM - 1) / cf.BM;
    p.tiles_n = (d->N + cf.BN - 1) / cf.BN;
    // Split K when the tiles cannot occupy the compute units, keeping at least
    // four k-tiles per split.
    const long long tiles = (long long)p.tiles_m * p.tiles_n * batch;
    const int cus = compute_units();
    int splits = 1;
    if (tiles < cus) {
        const long long want = (cus + tiles - 1) / tiles;
        const long long most = d->K / (4LL * cf.BK);
        splits = (int)std::max(1LL, std::min(want, most));
    }
    splits = std::max(1, std::min(splits, env_cfg("ORMI_GEMM_MAX_SPLITS", 16)));
    if (batch * splits > 65535) splits = 1;
    const int kps = ((d->K + splits - 1) / splits + cf.BK - 1) / cf.BK * cf.BK;
    splits = (d->K + kps - 1) / kps;
    p.splits = splits;
    p.k_per_split = kps;
    const size_t out_elems = (size_t)batch * d->M * d->N;
    // The epilogue runs inside the fp32 kernels of configurations 2 and 3
    // (the fp32 defaults) for shapes in whole tiles and the functions those
    // kernels are instantiated for (epi_in_store). Other kernels store the
    // plain product and the finish pass applies it: the direct-load 16-bit
    // kernels keep their epilogue arguments few (they are pinned in scalar
    // registers ahead of the main loop), and an epilogue in every unrolled
    // store loop of every configuration would multiply the library's code.
    const bool even = d->M % cf.BM == 0 && d->N % cf.BN == 0 && d->K % cf.BK == 0;
    const bool epi_in_kernel = !dma && f32 && (dma32 || id == 2 || id == 3) && even && epi_in_store(epi);
    const bool finish = splits > 1 || (!epi_in_kernel && epi.kind != ORMI_GEMM_EPI_NONE);
    if (finish) {
        void* ws = nullptr;
        rc = workspace(out_elems * splits * sizeof(float), &ws);
        if (rc != ORMI_HIP_OK) return rc;
        p.c = (float*)ws;
        p.epi = Epi{};
        p.epi.kind = ORMI_GEMM_EPI_NONE;
    }
    dim3 grid(p.tiles_m * p.tiles_n, 1, (unsigned)(batch * splits));
    // fp32 default configuration with more whole tiles than compute units, one
    // batch and no K split: one persistent work-group per compute unit walks
    // its tiles as one stream of k-tiles (ORMI_GEMM_PERSIST=0 turns it off).
    // An activation epilogue in the store keeps the one-tile kernel (=2 takes
    // it too): with the activations compiled into the loop's kernel, its main
    // loop measured 3% slower at K = 4096.
    const int persist_env = env_cfg("ORMI_GEMM_PERSIST", 1);
    const bool persist = dma32 && dma32_id == 1 && even && splits == 1 && batch == 1 && tiles > cus &&
                         persist_env != 0 && (p.epi.kind != ORMI_GEMM_EPI_UNARY || persist_env == 2);
    if (dma && d->dtype == ORMI_DTYPE_BF16) run_dma<TrBF16>(id, p, grid, a_kc, b_kc);
    else if (dma) run_dma<TrF16>(id, p, grid, a_kc, b_kc);
    else if (dma32 && persist) run32_dma_persist(p, cus, a_kc, b_kc);
    else if (dma32) run32_dma(id, p, grid, a_kc, b_kc, p.epi.kind != ORMI_GEMM_EPI_NONE);
    else if (f32 && p.epi.kind != ORMI_GEMM_EPI_NONE) run32_epi(id, p, grid, a_kc, b_kc);
    else if (f32) run32(id, p, grid, even, a_kc, b_kc);
    else if (d->dtype == ORMI_DTYPE_BF16) run16<TrBF16>(id, p, grid, even, a_kc, b_kc);
    else run16<TrF16>(id, p, grid, even, a_kc, b_kc);
    if (finish) launch_finish(d, p.c, splits, batch, epi);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(ORMI_HIP_ERR_RUNTIME, std::string("ormi_hip_gemm launch: ") + hipGetErrorString(e));
    return ORMI_HIP_OK;
}
}  // namespace ormi_hip

extern "C" int ormi_hip_gemm(const ormi_gemm_desc* d) { return gemm_run(d, nullptr, false); }

extern "C" int ormi_hip_gemm_ex(const ormi_gemm_desc* d, const ormi_gemm_epilogue* epi) { return gemm_run(d, epi, false); }

extern "C" int ormi_hip_gemm_ex_noalloc(const ormi_gemm_desc* d, const ormi_gemm_epilogue* epi) {
    return gemm_run(d, epi, true);
}

extern "C" int ormi_hip_gemm_pair(const ormi_gemm_desc* d0, const ormi_gemm_epilogue* e0, const ormi_gemm_desc* d1,
                                  const ormi_gemm_epilogue* e1, int* grouped) {
    return ormi_hip::gemm_pair(d0, e0, d1, e1, grouped);
}
