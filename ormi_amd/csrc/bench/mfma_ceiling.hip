// Matrix-core ceilings of this GPU, the denominators a GEMM's MFMA utilisation
// is judged against beside the datasheet peaks. Register-only loops of
// v_mfma_f32_32x32x16_bf16 and v_mfma_f32_32x32x2_f32 (the instructions the
// GEMM kernels use), 4 independent accumulators per wave, 1 or 2 waves per
// SIMD. Operands are either constant or change every instruction with values
// drawn from N(0, 1/64): matrix-core power, and so the clock the chip holds,
// depends on how many operand bits toggle, and a GEMM's operands toggle.
// Prints one JSON object per line. Built by ormi_amd/_build.py; run through
// `python3 bench.py --ceilings`.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define CHECK(x)                                                                  \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                   \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));          \
            std::exit(1);                                                         \
        }                                                                         \
    } while (0)

// fp32: 8 operand pairs per lane cycle through the 4 accumulators.
template <bool RAND>
__global__ __launch_bounds__(256) void mfma_f32(float* out, const float* in, int iters) {
    float av[8], bv[8];
    for (int i = 0; i < 8; ++i) {
        av[i] = in[(threadIdx.x * 16 + blockIdx.x * 7 + i) & 4095];
        bv[i] = in[(threadIdx.x * 16 + blockIdx.x * 7 + 8 + i) & 4095];
    }
    f32x16 acc[4];
    for (int j = 0; j < 4; ++j)
        for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(RAND ? av[u] : av[0], RAND ? bv[(u + j) & 7] : bv[0], acc[j], 0, 0, 0);
    }
    float s = 0.0f;
    for (int j = 0; j < 4; ++j)
        for (int i = 0; i < 16; ++i) s += acc[j][i];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

// bf16: 4 operand-vector pairs per lane.
template <bool RAND>
__global__ __launch_bounds__(256) void mfma_bf16(float* out, const float* in, int iters) {
    bf16x8 av[4], bv[4];
    for (int v = 0; v < 4; ++v)
        for (int i = 0; i < 8; ++i) {
            av[v][i] = (__bf16)in[(threadIdx.x * 64 + blockIdx.x * 5 + v * 8 + i) & 4095];
            bv[v][i] = (__bf16)in[(threadIdx.x * 64 + blockIdx.x * 5 + 32 + v * 8 + i) & 4095];
        }
    f32x16 acc[4];
    for (int j = 0; j < 4; ++j)
        for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(RAND ? av[u] : av[0], RAND ? bv[(u + j) & 3] : bv[0], acc[j], 0, 0, 0);
    }
    float s = 0.0f;
    for (int j = 0; j < 4; ++j)
        for (int i = 0; i < 16; ++i) s += acc[j][i];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

int main() {
    int cus = 0;
    hipDeviceProp_t prop;
    CHECK(hipGetDeviceProperties(&prop, 0));
    cus = prop.multiProcessorCount;
    float *out = nullptr, *in = nullptr;
    CHECK(hipMalloc(&out, (size_t)cus * 2 * 256 * sizeof(float)));
    CHECK(hipMalloc(&in, 4096 * sizeof(float)));
    // N(0, 1/64) by Box-Muller from a fixed LCG: the operand statistics of the
    // C4 benchmark's inputs.
    std::vector<float> h(4096);
    unsigned long long st = 12345;
    auto uni = [&] {
        st = st * 6364136223846793005ULL + 1442695040888963407ULL;
        return ((st >> 11) + 0.5) / 9007199254740992.0;
    };
    for (auto& x : h) x = (float)(std::sqrt(-2.0 * std::log(uni())) * std::cos(6.283185307179586 * uni()) / 8.0);
    CHECK(hipMemcpy(in, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));

    struct Case {
        const char* op;
        bool rand;
        void (*k)(float*, const float*, int);
        double flop_per_iter_per_wave;
        int iters;
    };
    const Case cases[] = {
        {"bf16_32x32x16", false, mfma_bf16<false>, 16.0 * 32768, 16000},
        {"bf16_32x32x16", true, mfma_bf16<true>, 16.0 * 32768, 16000},
        {"f32_32x32x2", false, mfma_f32<false>, 32.0 * 4096, 8000},
        {"f32_32x32x2", true, mfma_f32<true>, 32.0 * 4096, 8000},
    };
    for (int waves = 1; waves <= 2; ++waves) {
        for (const Case& c : cases) {
            const int blocks = cus * waves;  // 4 waves per block, one per SIMD
            hipLaunchKernelGGL(c.k, dim3(blocks), dim3(256), 0, 0, out, in, 64);
            CHECK(hipGetLastError());
            CHECK(hipDeviceSynchronize());
            float best = 1e30f;
            for (int r = 0; r < 3; ++r) {
                CHECK(hipEventRecord(e0));
                hipLaunchKernelGGL(c.k, dim3(blocks), dim3(256), 0, 0, out, in, c.iters);
                CHECK(hipEventRecord(e1));
                CHECK(hipEventSynchronize(e1));
                float ms = 0.0f;
                CHECK(hipEventElapsedTime(&ms, e0, e1));
                if (ms < best) best = ms;
            }
            const double flop = c.flop_per_iter_per_wave * c.iters * blocks * 4.0;
            std::printf("{\"op\": \"%s\", \"operands\": \"%s\", \"waves_per_simd\": %d, \"ms\": %.3f, \"TFLOP/s\": %.1f}\n", c.op,
                        c.rand ? "random N(0,1/64)" : "constant", waves, best, flop / best / 1e9);
            std::fflush(stdout);
        }
    }
    CHECK(hipFree(out));
    CHECK(hipFree(in));
    return 0;
}
