// fp32 GEMM with direct HBM->LDS loads (gfx950 global_load_lds_dwordx4) and a
// multi-stage LDS ring, for v_mfma_f32_32x32x2_f32.
//
// Each load instruction moves 64 lanes x 16 bytes into 1 KB of LDS in lane
// order, so tiles are unpadded; bank conflicts are avoided with XOR swizzles
// of the 16-byte chunk index. A k-tile is BK = 32 or 64 floats deep:
//   k-contiguous operand  [BMN][BK]  4*BK-byte rows, physical chunk = c ^ swz_k(row),
//       BK 32: swz_k(r) = (r & 7) ^ ((r >> 3) & 1); BK 64: swz_k(r) = r & 15:
//       the chunks one 16-byte fragment read takes from 16 consecutive rows
//       land on distinct banks;
//   mn-contiguous operand [BK][BMN]  BMN*4-byte k-rows, physical chunk = c ^ swz_mn(k),
//       swz_mn(k) = 8 * ((k >> 2) & 1): a fragment read takes 32 consecutive
//       floats of k-row k with lanes 0-31 and of k-row k + 4 with lanes 32-63;
//       the swizzle puts those two 128-byte runs in different halves of the
//       64 banks.
// Fragments: lane l of a 32-row (or 32-column) block holds 4 consecutive k of
// its row, k = 8 s + 4 (l / 32) + e for k-step s and element e; element e of
// the A and B fragments feeds one K=2 MFMA (TrF32::mma pairs them the same
// way). A k-contiguous fragment is one ds_read_b128; an mn-contiguous one is
// four dword reads down the k-rows (gfx950 has no 32-bit transpose read).
//
// Pipeline (STAGES k-tiles in LDS, KS = BK / 8 k-steps of 8 k per tile):
// during tile kt each wave issues its share of the loads of tile
// kt + STAGES - 1 into the stage tile kt - 1 used, spread over k-steps
// 0..KS-2 after single MFMAs; the fragment reads of the next k-step are spread
// the same way. Before the last k-step the wave waits until tile kt + 1 has
// landed (its later loads may stay in flight) and its own LDS reads are done,
// then a barrier publishes tile kt + 1 and frees tile kt's stage; the last
// k-step reads k-step 0 of tile kt + 1. Loads past
// the last tile re-read the last tile into a stage no step reads, so every
// tile issues the same number of loads and each wait count is a constant.
// K must be a multiple of BK; rows and columns past M / N are clamped on load
// (they only feed outputs that are not stored); an mn-contiguous operand needs
// its extent (M or N) to be a multiple of 4.
#include "gemm_mfma.h"

#pragma clang diagnostic ignored "-Winline-asm"

namespace ormi_hip {

namespace {

template <int BK>
__device__ __forceinline__ int swz_k32(int r) {
    static_assert(BK == 32 || BK == 64, "tile depth 32 or 64 floats");
    return BK == 32 ? (r & 7) ^ ((r >> 3) & 1) : r & 15;
}
__device__ __forceinline__ int swz_mn32(int k) { return ((k >> 2) & 1) << 3; }

// Direct loads of one operand's BK-deep k-tiles: per-lane byte offsets within
// a tile are fixed along k, so they are computed once; a k-tile costs one
// scalar base and one instruction per 1 KB segment.
template <int BMN, bool KC, int NW, int BK>
struct Dma32 {
    static constexpr int SEGS = BMN * BK * 4 / 1024;
    static constexpr int PER = SEGS / NW;
    static_assert(SEGS % NW == 0 && PER >= 1, "segments must split evenly over waves");
    unsigned voff[PER];

    __device__ __forceinline__ void init(long long s_mn, long long s_k, int mn0, int MN) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
        for (int s = 0; s < PER; ++s) {
            const int q = wave * PER + s;
            if constexpr (KC) {
                constexpr int CPR = BK / 4;  // chunks per row
                const int row = q * (64 / CPR) + lane / CPR;
                const int c = (lane % CPR) ^ swz_k32<BK>(row);
                const int mn = min(mn0 + row, MN - 1) - mn0;
                voff[s] = (unsigned)(((long long)mn * s_mn + c * 4) * 4);
            } else {
                constexpr int CPR = BMN / 4;   // chunks per k-row
                constexpr int RPS = 64 / CPR;  // k-rows per segment
                const int k = q * RPS + lane / CPR;
                const int c = (lane % CPR) ^ swz_mn32(k);
                const int mn = min(mn0 + c * 4, MN - 4) - mn0;
                voff[s] = (unsigned)(((long long)k * s_k + mn) * 4);
            }
        }
    }
    __device__ __forceinline__ static long long origin(long long s_mn, long long s_k, int mn0, int k0) {
        return KC ? ((long long)mn0 * s_mn + k0) * 4 : ((long long)k0 * s_k + mn0) * 4;
    }
    __device__ __forceinline__ static long long kstep(long long s_k) { return KC ? 4 * BK : 4 * BK * s_k; }

    // Issued as inline assembly so that the compiler's wait counting does not
    // make LDS reads of the current stage wait for these loads of a later one;
    // the kernel waits for them itself before the barrier that publishes them.
    __device__ __forceinline__ void issue_one(lds_char* lds, const char* base, int s) const {
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const unsigned dst = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds + (wave * PER + s) * 1024));
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"(voff[s]), "s"(base)
                     : "memory", "m0");
    }
};

__device__ __forceinline__ const char* uniform_ptr(const char* p) {
    const unsigned long long t = (unsigned long long)(uintptr_t)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)t);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(t >> 32));
    return (const char*)(((unsigned long long)hi << 32) | lo);
}

// Fragment of rows (or columns) [row0, row0 + 32), k-step s.
template <int BMN, bool KC, int BK>
__device__ __forceinline__ u32x4_t frag32(const lds_char* lds, int row0, int s) {
    const int lane = threadIdx.x & 63;
    if constexpr (KC) {
        const int row = row0 + (lane & 31);
        const int c = s * 2 + (lane >> 5);
        return *(const __attribute__((address_space(3))) u32x4_t*)(lds + row * (4 * BK) + ((c ^ swz_k32<BK>(row)) << 4));
    } else {
        const int n = row0 + (lane & 31);
        const int k = s * 8 + (lane >> 5) * 4;  // k .. k + 3 share one swizzle
        const __attribute__((address_space(3))) unsigned* f =
            (const __attribute__((address_space(3))) unsigned*)(lds + k * (BMN * 4) + (((n >> 2) ^ swz_mn32(k)) << 4) +
                                                                 ((n & 3) << 2));
        return u32x4_t{f[0], f[BMN], f[2 * BMN], f[3 * BMN]};
    }
}

template <int BM, int BN, int BK, int WGM, int WGN, bool A_KC, bool B_KC>
struct Il32 {
    static constexpr int NW = WGM * WGN, KS = BK / 8;
    static constexpr bool kAKC = A_KC, kBKC = B_KC;
    static constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
    static constexpr int A_BYTES = BM * BK * 4, STAGE = A_BYTES + BN * BK * 4;
    using PlanA = Dma32<BM, A_KC, NW, BK>;
    using PlanB = Dma32<BN, B_KC, NW, BK>;
    static constexpr int PA = PlanA::PER, PB = PlanB::PER, PER_TILE = PA + PB;
    static constexpr int NM = 4 * TM * TN;  // MFMAs per k-step
    static constexpr int NR = TM + TN;      // fragment reads per k-step

    // Loads of k-step s (0..KS-2): [s * PER_TILE / (KS - 1), (s + 1) * PER_TILE / (KS - 1)).
    static constexpr int load_lo(int s) { return s >= KS - 1 ? PER_TILE : s * PER_TILE / (KS - 1); }
    static constexpr int mem_ops(int s) { return NR + load_lo(s + 1) - load_lo(s); }

    // LA / LB: the load plans (PlanA / PlanB, or plans of the same extents for
    // another operand layout: issuing a load does not depend on the layout).
    template <int S, class LA, class LB>
    __device__ __forceinline__ static void mem_op(int o, u32x4_t (&fa)[TM], u32x4_t (&fb)[TN],
                                                  const lds_char* rs, int rks, int wm, int wn, lds_char* fs,
                                                  const char* ta, const char* tb, const LA& pa, const LB& pb) {
        // Reads in the order the next step's first MFMAs use them: A0, B0.., A1..
        if (o == 0) {
            fa[0] = frag32<BM, A_KC, BK>(rs, wm * WTM, rks);
        } else if (o <= TN) {
            fb[o - 1] = frag32<BN, B_KC, BK>(rs + A_BYTES, wn * WTN + (o - 1) * 32, rks);
        } else if (o < NR) {
            const int i = o - TN;
            fa[i] = frag32<BM, A_KC, BK>(rs, wm * WTM + i * 32, rks);
        } else {
            const int d = load_lo(S) + (o - NR);
            if (d < PA) pa.issue_one(fs, ta, d);
            else pb.issue_one(fs + A_BYTES, tb, d - PA);
        }
    }

    // MFMAs of one k-step, element-major (consecutive MFMAs on one
    // accumulator are TM * TN apart), each followed by its share of the
    // step's memory instructions.
    template <int S, class LA, class LB>
    __device__ __forceinline__ static void run(f32x16_t (&acc)[TM][TN], const u32x4_t (&ua)[TM],
                                               const u32x4_t (&ub)[TN], u32x4_t (&fa)[TM], u32x4_t (&fb)[TN],
                                               const lds_char* rs, int rks, int wm, int wn, lds_char* fs,
                                               const char* ta, const char* tb, const LA& pa, const LB& pb) {
        constexpr int NO = mem_ops(S);
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            const int e = n / (TM * TN), ij = n % (TM * TN), i = ij / TN, j = ij % TN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(ua[i][e]), __uint_as_float(ub[j][e]),
                                                             acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int o = n * NO / NM; o < (n + 1) * NO / NM; ++o) {
                mem_op<S, LA, LB>(o, fa, fb, rs, rks, wm, wn, fs, ta, tb, pa, pb);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
};

// Runs the k-steps S..KS-2 of a tile (fragments alternate between the two
// register sets), all reading the current stage.
template <typename St, int S>
struct Steps {
    template <typename... Args>
    __device__ __forceinline__ static void run(f32x16_t (&acc)[St::TM][St::TN], u32x4_t (&fa)[2][St::TM],
                                               u32x4_t (&fb)[2][St::TN], const lds_char* cur, Args... args) {
        if constexpr (S < St::KS - 1) {
            St::template run<S>(acc, fa[S & 1], fb[S & 1], fa[(S + 1) & 1], fb[(S + 1) & 1], cur, S + 1, args...);
            Steps<St, S + 1>::run(acc, fa, fb, cur, args...);
        }
    }
};

// EPI: the element-wise epilogue p.epi is applied in the store (only for
// shapes in whole tiles without a K split; the host checks).
template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, bool A_KC, bool B_KC, bool EPI>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_f32dma_kernel(GemmParams p) {
    static_assert(STAGES >= 2 && STAGES <= 5, "2 to 5 stages");
    using St = Il32<BM, BN, BK, WGM, WGN, A_KC, B_KC>;
    constexpr int TM = St::TM, TN = St::TN, WTM = St::WTM, WTN = St::WTN, KS = St::KS;
    constexpr int A_BYTES = St::A_BYTES, STAGE = St::STAGE, PER_TILE = St::PER_TILE;
    __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE];

    // Tile index: XCD-aware remap, then groups of 4 tile rows.
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
    long long a_off = 0, b_off = 0, d_off = 0;
    const long long c_off = ((long long)split * p.batch + bidx) * p.M * p.N;
    for (int d = p.batch_ndim - 1; d >= 0; --d) {
        const int coord = bidx % p.batch_shape[d];
        bidx /= p.batch_shape[d];
        a_off += coord * p.a_bs[d];
        b_off += coord * p.b_bs[d];
        d_off += coord * p.epi.d_bs[d];
    }
    float* c = p.c + c_off;
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int KT = kend > kbeg ? (kend - kbeg) / BK : 0;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

    typename St::PlanA pa;
    typename St::PlanB pb;
    pa.init(p.a_sm, p.a_sk, m0, p.M);
    pb.init(p.b_sn, p.b_sk, n0, p.N);
    const char* ta = p.a + a_off * 4 + St::PlanA::origin(p.a_sm, p.a_sk, m0, kbeg);
    const char* tb = p.b + b_off * 4 + St::PlanB::origin(p.b_sn, p.b_sk, n0, kbeg);
    const long long a_step = St::PlanA::kstep(p.a_sk), b_step = St::PlanB::kstep(p.b_sk);
    lds_char* const lds = (lds_char*)smem;
    // Epilogue arguments are loaded before the loop: a scalar load in flight
    // there would make every LDS wait in the loop drain completely.
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
            const char* ua = uniform_ptr(ta);
            const char* ub = uniform_ptr(tb);
#pragma unroll
            for (int d = 0; d < St::PA; ++d) pa.issue_one(lds + s * STAGE, ua, d);
#pragma unroll
            for (int d = 0; d < St::PB; ++d) pb.issue_one(lds + s * STAGE + A_BYTES, ub, d);
            if (s + 1 < KT) {
                ta += a_step;
                tb += b_step;
            }
        }
        wait_vmcnt<(STAGES - 2) * PER_TILE>();
        lds_barrier();
        u32x4_t fa[2][TM], fb[2][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[0][i] = frag32<BM, A_KC, BK>(lds, wm * WTM + i * 32, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[0][j] = frag32<BN, B_KC, BK>(lds + A_BYTES, wn * WTN + j * 32, 0);

        int stage = 0, free_stage = STAGES - 1;
        for (int kt = 0; kt < KT; ++kt) {
            const int next = stage + 1 == STAGES ? 0 : stage + 1;
            const lds_char* cur = lds + stage * STAGE;
            lds_char* fs = lds + free_stage * STAGE;
            const char* ua = uniform_ptr(ta);
            const char* ub = uniform_ptr(tb);
            static_assert(KS % 2 == 0, "the last k-step's fragments are in the second register set");
            Steps<St, 0>::run(acc, fa, fb, cur, wm, wn, fs, ua, ub, pa, pb);
            // Tile kt+1 landed (this tile's loads, for tile kt+STAGES-1, and
            // the STAGES-3 tiles before it may stay in flight) and this wave's
            // reads of tile kt are done; the barrier publishes kt+1 to every
            // wave and frees tile kt's stage for the loads of tile kt+1.
            wait_vmcnt_lds<(STAGES - 2) * PER_TILE>();
            lds_barrier();
            St::template run<KS - 1>(acc, fa[1], fb[1], fa[0], fb[0], lds + next * STAGE, 0, wm, wn, fs, ua, ub, pa, pb);
            if (kt + STAGES < KT) {
                ta += a_step;
                tb += b_step;
            }
            stage = next;
            free_stage = free_stage + 1 == STAGES ? 0 : free_stage + 1;
        }
        // No load may still be writing this workgroup's LDS when it exits,
        // and the epilogue's loads start from an empty counter.
        wait_vmcnt<0>();
    }

    if constexpr (EPI) {
        float dv[TM][TN][16];
        epi_tile<TM, TN, false>(p.epi, p.epi.s ? *p.epi.s : 0.0f, c, p.epi.aux ? p.epi.aux + c_off : nullptr, p.epi.d + d_off, p.N, m0 + wm * WTM,
                                n0 + wn * WTN, acc, dv, epi_reads_d(p.epi));
        return;
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

// Persistent form of gemm_f32dma_kernel for an output in whole tiles, one
// batch, no K split and more tiles than work-groups (one per compute unit):
// work-group b takes tiles b, b + G, b + 2G, ... (G work-groups, same tile
// order as the one-tile kernel) and runs them as one stream of k-tiles
// through the same LDS ring, so the loads of a tile's first k-tiles are in
// flight while the previous tile finishes, and its stores drain while the
// next tile's MFMAs run. The per-launch fill, the epilogue's latency and the
// work-group turnover are paid once per work-group instead of once per tile.
// EK: the epilogue kind compiled in (ORMI_GEMM_EPI_*; NONE: plain stores).
template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, bool A_KC, bool B_KC, int EK>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_f32dma_persist_kernel(GemmParams p) {
    constexpr bool EPI = EK != ORMI_GEMM_EPI_NONE;
    static_assert(STAGES >= 2 && STAGES <= 5, "2 to 5 stages");
    using St = Il32<BM, BN, BK, WGM, WGN, A_KC, B_KC>;
    constexpr int TM = St::TM, TN = St::TN, WTM = St::WTM, WTN = St::WTN, KS = St::KS;
    constexpr int A_BYTES = St::A_BYTES, STAGE = St::STAGE, PER_TILE = St::PER_TILE;
    __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE];

    const int T = p.tiles_m * p.tiles_n, G = gridDim.x;
    const int mine = (T - (int)blockIdx.x + G - 1) / G;  // tiles of this work-group
    const int KT = p.K / BK;
    const long long GT = (long long)mine * KT;  // k-tiles in its stream
    // Tile i of this work-group: XCD-aware remap, then groups of 4 tile rows.
    auto tile_origin = [&](int i, int& m0, int& n0) {
        int t = (int)blockIdx.x + i * G;
        if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
        constexpr int GROUP = 4;
        const int group_size = GROUP * p.tiles_n;
        const int g = t / group_size, first_m = g * GROUP;
        const int gm = min(p.tiles_m - first_m, GROUP);
        m0 = (first_m + (t % group_size) % gm) * BM;
        n0 = ((t % group_size) / gm) * BN;
    };

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    typename St::PlanA pa;
    typename St::PlanB pb;
    // Whole tiles: a tile's per-lane offsets do not depend on where it lies.
    pa.init(p.a_sm, p.a_sk, 0, p.M);
    pb.init(p.b_sn, p.b_sk, 0, p.N);
    const long long a_step = St::PlanA::kstep(p.a_sk), b_step = St::PlanB::kstep(p.b_sk);
    // Next k-tile of the stream to load: tile li, k-tile lkt, at ta / tb; it
    // stays on the last one once the stream is exhausted.
    int li = 0, lkt = 0;
    const char* ta;
    const char* tb;
    auto set_load_tile = [&](int i) {
        int m0, n0;
        tile_origin(i, m0, n0);
        ta = p.a + St::PlanA::origin(p.a_sm, p.a_sk, m0, 0);
        tb = p.b + St::PlanB::origin(p.b_sn, p.b_sk, n0, 0);
    };
    auto advance = [&]() {
        if (lkt + 1 < KT) {
            ++lkt;
            ta += a_step;
            tb += b_step;
        } else if (li + 1 < mine) {
            ++li;
            lkt = 0;
            set_load_tile(li);
        }
    };
    set_load_tile(0);
    lds_char* const lds = (lds_char*)smem;
    float* const c = p.c;
    // The epilogue's scale is read once, before the loop: a load of it at
    // each tile's end would make the compiler drain every outstanding load.
    const float sv =
        EPI && p.epi.s ? __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(*p.epi.s))) : 0.0f;
    asm volatile("" ::"s"(c), "s"(p.M), "s"(p.N), "s"(sv));

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if (GT > 0) {
#pragma unroll
        for (int s = 0; s < STAGES - 1; ++s) {
            const char* ua = uniform_ptr(ta);
            const char* ub = uniform_ptr(tb);
#pragma unroll
            for (int d = 0; d < St::PA; ++d) pa.issue_one(lds + s * STAGE, ua, d);
#pragma unroll
            for (int d = 0; d < St::PB; ++d) pb.issue_one(lds + s * STAGE + A_BYTES, ub, d);
            if (s + 1 < GT) advance();
        }
        wait_vmcnt<(STAGES - 2) * PER_TILE>();
        lds_barrier();
        u32x4_t fa[2][TM], fb[2][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[0][i] = frag32<BM, A_KC, BK>(lds, wm * WTM + i * 32, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[0][j] = frag32<BN, B_KC, BK>(lds + A_BYTES, wn * WTN + j * 32, 0);

        int stage = 0, free_stage = STAGES - 1, tile = 0, kt = 0, cm0, cn0;
        tile_origin(0, cm0, cn0);
        for (long long g = 0; g < GT; ++g) {
            const int next = stage + 1 == STAGES ? 0 : stage + 1;
            const lds_char* cur = lds + stage * STAGE;
            lds_char* fs = lds + free_stage * STAGE;
            const char* ua = uniform_ptr(ta);
            const char* ub = uniform_ptr(tb);
            Steps<St, 0>::run(acc, fa, fb, cur, wm, wn, fs, ua, ub, pa, pb);
            wait_vmcnt_lds<(STAGES - 2) * PER_TILE>();
            lds_barrier();
            St::template run<KS - 1>(acc, fa[1], fb[1], fa[0], fb[0], lds + next * STAGE, 0, wm, wn, fs, ua, ub, pa, pb);
            // Keeps the step's fragment reads among its MFMAs: without it the
            // compiler sinks them below the branches that follow, and the next
            // k-tile's first MFMAs wait out their whole latency.
            asm volatile("" ::: "memory");
            if (g + STAGES < GT) advance();
            stage = next;
            free_stage = free_stage + 1 == STAGES ? 0 : free_stage + 1;
            if (++kt == KT) {
                // Tile done: its stores go out while the next tile's k-tiles,
                // already loading, run on fresh accumulators.
                if constexpr (EPI) {
                    float dv[TM][TN][16];
                    epi_tile<TM, TN, false, EK>(p.epi, sv, c, p.epi.aux, p.epi.d, p.N, cm0 + wm * WTM, cn0 + wn * WTN,
                                                acc, dv, epi_reads_d(p.epi));
                } else {
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            const int col = cn0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                const int row = cm0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                                c[(long long)row * p.N + col] = acc[i][j][r];
                            }
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
                kt = 0;
                if (++tile < mine) tile_origin(tile, cm0, cn0);
            }
        }
        // No load may still be writing this workgroup's LDS when it exits.
        wait_vmcnt<0>();
    }
}

// Two independent products in one persistent launch (the dX and dW GEMMs of
// one layer's backward read the same dZ and nothing of each other). Problem q
// has its own operands, layouts (A_KCq / B_KCq), K and epilogue (EKq), each in
// whole tiles with one batch and no K split. The tiles of problem 0, then of
// problem 1, form one list; work-group b takes entries b, b + G, b + 2G, ...,
// so it runs its problem-0 tiles first, then its problem-1 tiles, as one
// stream of k-tiles through one LDS ring: the first k-tiles of its problem-1
// stream are loading while its last problem-0 tile finishes. A tile is
// computed exactly as gemm_f32dma_kernel / gemm_f32dma_persist_kernel compute
// it (the same k-steps in the same order, the same epilogue), so each output
// is bit-identical to its product's own launch.
template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, bool A_KC0, bool B_KC0, int EK0, bool A_KC1,
          bool B_KC1, int EK1>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_f32dma_pair_kernel(GemmParams p0, GemmParams p1) {
    static_assert(STAGES >= 2 && STAGES <= 5, "2 to 5 stages");
    using St0 = Il32<BM, BN, BK, WGM, WGN, A_KC0, B_KC0>;
    using St1 = Il32<BM, BN, BK, WGM, WGN, A_KC1, B_KC1>;
    constexpr int TM = St0::TM, TN = St0::TN, WTM = St0::WTM, WTN = St0::WTN, KS = St0::KS;
    constexpr int A_BYTES = St0::A_BYTES, STAGE = St0::STAGE, PER_TILE = St0::PER_TILE;
    static_assert(St1::STAGE == STAGE && St1::PER_TILE == PER_TILE && St1::PA == St0::PA, "one ring for both");
    __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE];

    const int T0 = p0.tiles_m * p0.tiles_n, T1 = p1.tiles_m * p1.tiles_n, G = gridDim.x;
    const int b = blockIdx.x;
    const int mine = (T0 + T1 - b + G - 1) / G;           // list entries of this work-group
    const int mine0 = b < T0 ? (T0 - b + G - 1) / G : 0;  // ... of problem 0, which come first
    const int KT0 = p0.K / BK, KT1 = p1.K / BK;
    const long long GT0 = (long long)mine0 * KT0, GT = GT0 + (long long)(mine - mine0) * KT1;
    // Problem 1's value if q, else problem 0's. By value: a conditional over
    // two lvalues selects between their addresses, which keeps both in
    // scratch memory.
    auto pick = [](bool q, auto v0, auto v1) { return q ? v1 : v0; };
    // Entry i of this work-group: its problem's tile index, XCD-aware remap,
    // then groups of 4 tile rows (the one-problem kernels' order).
    auto tile_origin = [&](int i, int& m0, int& n0) {
        const int u = b + i * G;
        const bool q = u >= T0;
        const int T = pick(q, T0, T1), tiles_m = pick(q, p0.tiles_m, p1.tiles_m), tiles_n = pick(q, p0.tiles_n, p1.tiles_n);
        int t = q ? u - T0 : u;
        if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
        constexpr int GROUP = 4;
        const int group_size = GROUP * tiles_n;
        const int g = t / group_size, first_m = g * GROUP;
        const int gm = min(tiles_m - first_m, GROUP);
        m0 = (first_m + (t % group_size) % gm) * BM;
        n0 = ((t % group_size) / gm) * BN;
    };

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    // Per-lane load offsets of each problem's layouts (whole tiles: independent
    // of the tile). They never change: each stretch of the stream below loads
    // with one problem's pair of them, so no per-lane value is reassigned in a
    // loop (a reassigned one is copied between registers on every k-tile).
    typename St0::PlanA pa0;
    typename St0::PlanB pb0;
    typename St1::PlanA pa1;
    typename St1::PlanB pb1;
    pa0.init(p0.a_sm, p0.a_sk, 0, p0.M);
    pb0.init(p0.b_sn, p0.b_sk, 0, p0.N);
    pa1.init(p1.a_sm, p1.a_sk, 0, p1.M);
    pb1.init(p1.b_sn, p1.b_sk, 0, p1.N);
    // Next k-tile of the stream to load: entry li, k-tile lkt of it, at ta /
    // tb; it stays on the last one once the stream is exhausted. All uniform.
    int li = 0, lkt = 0;
    const char* ta;
    const char* tb;
    auto set_load_tile = [&](int i) {
        int m0, n0;
        tile_origin(i, m0, n0);
        if (b + i * G < T0) {
            ta = p0.a + St0::PlanA::origin(p0.a_sm, p0.a_sk, m0, 0);
            tb = p0.b + St0::PlanB::origin(p0.b_sn, p0.b_sk, n0, 0);
        } else {
            ta = p1.a + St1::PlanA::origin(p1.a_sm, p1.a_sk, m0, 0);
            tb = p1.b + St1::PlanB::origin(p1.b_sn, p1.b_sk, n0, 0);
        }
    };
    // One k-tile on, within the load stream's current problem Q (known where
    // it is called, so its depth and steps are constants there), or on to the
    // next entry, which may be the other problem's.
    auto advance = [&](auto q_tag) __attribute__((always_inline)) {
        constexpr int Q = decltype(q_tag)::value;
        if (lkt + 1 < (Q ? KT1 : KT0)) {
            ++lkt;
            ta += Q ? St1::PlanA::kstep(p1.a_sk) : St0::PlanA::kstep(p0.a_sk);
            tb += Q ? St1::PlanB::kstep(p1.b_sk) : St0::PlanB::kstep(p0.b_sk);
        } else if (li + 1 < mine) {
            ++li;
            lkt = 0;
            set_load_tile(li);
        }
    };
    set_load_tile(0);
    lds_char* const lds = (lds_char*)smem;
    // The epilogues' scales are read once, before the loop (a load of one at a
    // tile's end would make the compiler drain every outstanding load).
    const float sv0 = EK0 != ORMI_GEMM_EPI_NONE && p0.epi.s
                          ? __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(*p0.epi.s))) : 0.0f;
    const float sv1 = EK1 != ORMI_GEMM_EPI_NONE && p1.epi.s
                          ? __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(*p1.epi.s))) : 0.0f;
    asm volatile("" ::"s"(p0.c), "s"(p0.N), "s"(sv0), "s"(p1.c), "s"(p1.N), "s"(sv1));

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    if (GT == 0) return;

    // Prologue: k-tiles 0 .. STAGES-2, of either problem.
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) {
        const char* ua = uniform_ptr(ta);
        const char* ub = uniform_ptr(tb);
        if (b + li * G < T0) {
#pragma unroll
            for (int d = 0; d < St0::PA; ++d) pa0.issue_one(lds + s * STAGE, ua, d);
#pragma unroll
            for (int d = 0; d < St0::PB; ++d) pb0.issue_one(lds + s * STAGE + A_BYTES, ub, d);
            if (s + 1 < GT) advance(FnConst<0>{});
        } else {
#pragma unroll
            for (int d = 0; d < St1::PA; ++d) pa1.issue_one(lds + s * STAGE, ua, d);
#pragma unroll
            for (int d = 0; d < St1::PB; ++d) pb1.issue_one(lds + s * STAGE + A_BYTES, ub, d);
            if (s + 1 < GT) advance(FnConst<1>{});
        }
    }
    wait_vmcnt<(STAGES - 2) * PER_TILE>();
    lds_barrier();
    u32x4_t fa[2][TM], fb[2][TN];
    // Fragments of k-step 0 of the k-tile in stage `at`, in problem St's layouts.
    auto first_frags = [&](auto st, int at) __attribute__((always_inline)) {
        using S = decltype(st);
        const lds_char* cur = lds + at * STAGE;
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[0][i] = frag32<BM, S::kAKC, BK>(cur, wm * WTM + i * 32, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[0][j] = frag32<BN, S::kBKC, BK>(cur + A_BYTES, wn * WTN + j * 32, 0);
    };
    int stage = 0, free_stage = STAGES - 1;
    // Compute-side position in the current problem: entry `tile`, k-tile kt,
    // output origin (cm0, cn0).
    int tile = 0, kt = 0, cm0 = 0, cn0 = 0;
    // Stream steps [g_lo, g_hi): k-tiles of problem St (epilogue kind EK,
    // params p, KT k-tiles per tile), loading problem LQ's k-tiles with its
    // plans la / lb.
    auto run = [&](auto st, auto ek, const GemmParams& p, float sv, int KT, auto lq, const auto& la, const auto& lb,
                   long long g_lo, long long g_hi) __attribute__((always_inline)) {
        using St = decltype(st);
        constexpr int EK = decltype(ek)::value;
        for (long long g = g_lo; g < g_hi; ++g) {
            const int next = stage + 1 == STAGES ? 0 : stage + 1;
            const lds_char* cur = lds + stage * STAGE;
            lds_char* fs = lds + free_stage * STAGE;
            const char* ua = uniform_ptr(ta);
            const char* ub = uniform_ptr(tb);
            Steps<St, 0>::run(acc, fa, fb, cur, wm, wn, fs, ua, ub, la, lb);
            wait_vmcnt_lds<(STAGES - 2) * PER_TILE>();
            lds_barrier();
            St::template run<KS - 1>(acc, fa[1], fb[1], fa[0], fb[0], lds + next * STAGE, 0, wm, wn, fs, ua, ub, la, lb);
            asm volatile("" ::: "memory");
            if (g + STAGES < GT) advance(lq);
            stage = next;
            free_stage = free_stage + 1 == STAGES ? 0 : free_stage + 1;
            if (++kt == KT) {
                if constexpr (EK != ORMI_GEMM_EPI_NONE) {
                    float dv[TM][TN][16];
                    epi_tile<TM, TN, false, EK>(p.epi, sv, p.c, p.epi.aux, p.epi.d, p.N, cm0 + wm * WTM, cn0 + wn * WTN,
                                                acc, dv, epi_reads_d(p.epi));
                } else {
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            const int col = cn0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                const int row = cm0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                                p.c[(long long)row * p.N + col] = acc[i][j][r];
                            }
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
                kt = 0;
                if (++tile < mine) tile_origin(tile, cm0, cn0);
            }
        }
    };
    // Step g loads k-tile min(g + STAGES - 1, GT - 1): from g1 on, problem 1's.
    const long long g1 = GT > GT0 ? max(0LL, GT0 - (STAGES - 1)) : GT0;
    if (GT0 > 0) {
        first_frags(St0{}, 0);
        tile_origin(0, cm0, cn0);
        run(St0{}, FnConst<EK0>{}, p0, sv0, KT0, FnConst<0>{}, pa0, pb0, 0, g1);
        run(St0{}, FnConst<EK0>{}, p0, sv0, KT0, FnConst<1>{}, pa1, pb1, g1, GT0);
    }
    if (GT > GT0) {
        // The last problem-0 step read k-step 0 of this k-tile in problem 0's
        // layouts; the k-tile has landed (the barrier before that step), so
        // read it again in problem 1's.
        first_frags(St1{}, stage);
        tile = mine0;
        kt = 0;
        tile_origin(tile, cm0, cn0);
        run(St1{}, FnConst<EK1>{}, p1, sv1, KT1, FnConst<1>{}, pa1, pb1, GT0, GT);
    }
    // No load may still be writing this workgroup's LDS when it exits.
    wait_vmcnt<0>();
}

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES>
struct F32DmaLauncher {
    template <bool A_KC, bool B_KC>
    static void go(const GemmParams& p, dim3 grid, bool epi) {
        if (epi) gemm_f32dma_kernel<BM, BN, BK, WGM, WGN, STAGES, A_KC, B_KC, true><<<grid, 64 * WGM * WGN>>>(p);
        else gemm_f32dma_kernel<BM, BN, BK, WGM, WGN, STAGES, A_KC, B_KC, false><<<grid, 64 * WGM * WGN>>>(p);
    }
    static void run(const GemmParams& p, dim3 grid, bool a_kc, bool b_kc, bool epi) {
        if (a_kc && b_kc) go<true, true>(p, grid, epi);
        else if (a_kc) go<true, false>(p, grid, epi);
        else if (b_kc) go<false, true>(p, grid, epi);
        else go<false, false>(p, grid, epi);
    }
    template <bool A_KC, bool B_KC>
    static void go_persist(const GemmParams& p, int groups) {
        constexpr int NT = 64 * WGM * WGN;
        switch (p.epi.kind) {
            case ORMI_GEMM_EPI_ADD:
                gemm_f32dma_persist_kernel<BM, BN, BK, WGM, WGN, STAGES, A_KC, B_KC, ORMI_GEMM_EPI_ADD><<<groups, NT>>>(p);
                break;
            case ORMI_GEMM_EPI_UNARY:
                gemm_f32dma_persist_kernel<BM, BN, BK, WGM, WGN, STAGES, A_KC, B_KC, ORMI_GEMM_EPI_UNARY><<<groups, NT>>>(p);
                break;
            case ORMI_GEMM_EPI_MUL_FN_D:
                gemm_f32dma_persist_kernel<BM, BN, BK, WGM, WGN, STAGES, A_KC, B_KC, ORMI_GEMM_EPI_MUL_FN_D><<<groups, NT>>>(p);
                break;
            default:
                gemm_f32dma_persist_kernel<BM, BN, BK, WGM, WGN, STAGES, A_KC, B_KC, ORMI_GEMM_EPI_NONE><<<groups, NT>>>(p);
        }
    }
    static void run_persist(const GemmParams& p, int groups, bool a_kc, bool b_kc) {
        if (a_kc && b_kc) go_persist<true, true>(p, groups);
        else if (a_kc) go_persist<true, false>(p, groups);
        else if (b_kc) go_persist<false, true>(p, groups);
        else go_persist<false, false>(p, groups);
    }
};

}  // namespace

// Direct-load fp32 configurations (tile, waves, depth, stages, LDS):
//   0: 128x128, 2x2 waves (64x64 per wave), BK 32, 4 stages (128 KB)
//   1: 128x128, 2x4 waves (64x32 per wave), BK 32, 4 stages (128 KB)
//   2: 128x256, 2x2 waves (64x128 per wave), BK 32, 3 stages (144 KB)
//   3: 128x128, 2x2 waves, BK 32, 2 stages (64 KB: two work-groups per CU)
//   4: 128x128, 2x2 waves, BK 64, 2 stages (128 KB)
//   5: 128x128, 2x4 waves, BK 64, 2 stages (128 KB)
//   6: 128x64,  2x2 waves (64x32 per wave), BK 32, 4 stages (96 KB)
//   7: 64x128,  2x2 waves (32x64 per wave), BK 32, 4 stages (96 KB)
//   8: 128x64,  2x2 waves, BK 32, 5 stages (120 KB)
//   9: 128x64,  2x2 waves, BK 64, 3 stages (144 KB)
// Configuration 1 is the default (ORMI_GEMM_F32_DMA_CFG selects another;
// out-of-range ids select it too).
void cfg32_dma(int id, int* bm, int* bn, int* bk) {
    if (id < 0 || id > 9) id = 1;
    *bm = id == 7 ? 64 : 128;
    *bn = id == 2 ? 256 : id == 6 || id == 8 || id == 9 ? 64 : 128;
    *bk = id == 4 || id == 5 || id == 9 ? 64 : 32;
}
void run32_dma_persist(const GemmParams& p, int groups, bool a_kc, bool b_kc) {
    F32DmaLauncher<128, 128, 32, 2, 4, 4>::run_persist(p, groups, a_kc, b_kc);
}

namespace {
template <int EK0, int EK1>
void launch_pair(const GemmParams& p0, const GemmParams& p1, int groups) {
    gemm_f32dma_pair_kernel<128, 128, 32, 2, 4, 4, true, true, EK0, false, false, EK1><<<groups, 512>>>(p0, p1);
}
}  // namespace

// The layouts and epilogues one layer's backward produces: problem 0 is
// dZ Wᵀ (both operands k-contiguous), plain or with the activation's
// derivative in the store (MUL_FN_D); problem 1 is Xᵀ dZ (both operands
// mn-contiguous), plain or with the SGD update in the store (ADD).
bool run32_dma_pair(const GemmParams& p0, bool a_kc0, bool b_kc0, const GemmParams& p1, bool a_kc1, bool b_kc1,
                    int groups) {
    if (!(a_kc0 && b_kc0 && !a_kc1 && !b_kc1)) return false;
    const int k0 = p0.epi.kind, k1 = p1.epi.kind;
    if (k0 != ORMI_GEMM_EPI_NONE && k0 != ORMI_GEMM_EPI_MUL_FN_D) return false;
    if (k1 != ORMI_GEMM_EPI_NONE && k1 != ORMI_GEMM_EPI_ADD) return false;
    if (k0 == ORMI_GEMM_EPI_NONE && k1 == ORMI_GEMM_EPI_NONE) launch_pair<ORMI_GEMM_EPI_NONE, ORMI_GEMM_EPI_NONE>(p0, p1, groups);
    else if (k0 == ORMI_GEMM_EPI_NONE) launch_pair<ORMI_GEMM_EPI_NONE, ORMI_GEMM_EPI_ADD>(p0, p1, groups);
    else if (k1 == ORMI_GEMM_EPI_NONE) launch_pair<ORMI_GEMM_EPI_MUL_FN_D, ORMI_GEMM_EPI_NONE>(p0, p1, groups);
    else launch_pair<ORMI_GEMM_EPI_MUL_FN_D, ORMI_GEMM_EPI_ADD>(p0, p1, groups);
    return true;
}
void run32_dma(int id, const GemmParams& p, dim3 grid, bool a_kc, bool b_kc, bool epi) {
    if (id < 0 || id > 9) id = 1;
    switch (id) {
        case 0: F32DmaLauncher<128, 128, 32, 2, 2, 4>::run(p, grid, a_kc, b_kc, epi); break;
        case 2: F32DmaLauncher<128, 256, 32, 2, 2, 3>::run(p, grid, a_kc, b_kc, epi); break;
        case 3: F32DmaLauncher<128, 128, 32, 2, 2, 2>::run(p, grid, a_kc, b_kc, epi); break;
        case 4: F32DmaLauncher<128, 128, 64, 2, 2, 2>::run(p, grid, a_kc, b_kc, epi); break;
        case 5: F32DmaLauncher<128, 128, 64, 2, 4, 2>::run(p, grid, a_kc, b_kc, epi); break;
        case 6: F32DmaLauncher<128, 64, 32, 2, 2, 4>::run(p, grid, a_kc, b_kc, epi); break;
        case 7: F32DmaLauncher<64, 128, 32, 2, 2, 4>::run(p, grid, a_kc, b_kc, epi); break;
        case 8: F32DmaLauncher<128, 64, 32, 2, 2, 5>::run(p, grid, a_kc, b_kc, epi); break;
        case 9: F32DmaLauncher<128, 64, 64, 2, 2, 3>::run(p, grid, a_kc, b_kc, epi); break;
        default: F32DmaLauncher<128, 128, 32, 2, 4, 4>::run(p, grid, a_kc, b_kc, epi); break;
    }
}

}  // namespace ormi_hip
