// gemm_mfma_kernel instantiations that apply the element-wise epilogue in
// their store (fp32 configurations 2 and 3, the fp32 defaults, for shapes in
// whole tiles; ragged shapes take the finish pass). Kept apart
// from gemm.hip so the two translation units compile in parallel: the
// epilogue's functions, inlined into each fully unrolled store loop, make
// these the slowest kernels to compile.
#include "gemm_mfma.h"

namespace ormi_hip {

template <int BM, int BN, int WGM, int WGN>
struct EpiLauncher {
    template <bool A_KC, bool B_KC>
    static void go(const GemmParams& p, dim3 grid) {
        gemm_mfma_kernel<TrF32, BM, BN, 32, WGM, WGN, A_KC, B_KC, true, true><<<grid, 64 * WGM * WGN>>>(p);
    }
    static void run(const GemmParams& p, dim3 grid, bool a_kc, bool b_kc) {
        if (a_kc && b_kc) go<true, true>(p, grid);
        else if (a_kc) go<true, false>(p, grid);
        else if (b_kc) go<false, true>(p, grid);
        else go<false, false>(p, grid);
    }
};

void run32_epi(int id, const GemmParams& p, dim3 grid, bool a_kc, bool b_kc) {
    if (id == 3) EpiLauncher<128, 128, 2, 4>::run(p, grid, a_kc, b_kc);
    else EpiLauncher<128, 256, 2, 4>::run(p, grid, a_kc, b_kc);
}

}  // namespace ormi_hip
