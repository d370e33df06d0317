/*
 * ormi_hip.h — C ABI of libormi_hip.so, the MI355X (gfx950) device layer.
 *
 * The host C++ core (graph, autograd, fusion scheduler, hipRTC code generator)
 * reaches the GPU only through these functions. No C++ or torch types cross
 * this boundary: plain pointers, sizes and small POD descriptors.
 *
 * Conventions
 *   - Every function returns ORMI_HIP_OK (0) on success or a nonzero ORMI_HIP_ERR_*
 *     code; ormi_hip_last_error() then returns a message (thread-local).
 *   - All device work is ordered on the device's null stream, as the reference
 *     launches on the legacy default stream (csrc/backend/cuda/jit.cu:40).
 *     Copies to the host synchronize (csrc/backend/cuda/allocator.cu:89-91).
 *   - Device pointers belong to the caller. Compiled modules and kernel
 *     handles belong to the library's cache and live until process exit.
 *   - Memory entry points are thread-safe; launches are issued in call order
 *     (queued launches included: see ormi_hip_launch_queued).
 */
#ifndef ORMI_HIP_H
#define ORMI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORMI_HIP_OK               0
#define ORMI_HIP_ERR_RUNTIME      1  /* a HIP runtime call failed               */
#define ORMI_HIP_ERR_NO_DEVICE    2  /* no usable GPU in this process           */
#define ORMI_HIP_ERR_INVALID      3  /* bad argument (null, size, shape, dtype)  */
#define ORMI_HIP_ERR_COMPILE      4  /* hipRTC rejected the source              */
#define ORMI_HIP_ERR_UNSUPPORTED  5  /* valid request this build does not cover */

/* Element type codes; the numbering is ormi::DType's. */
#define ORMI_DTYPE_F32   0
#define ORMI_DTYPE_I32   1
#define ORMI_DTYPE_BOOL  2
#define ORMI_DTYPE_BF16  3
#define ORMI_DTYPE_F16   4
#define ORMI_DTYPE_I64   5

/* ---------------------------------------------------------------- device --
 * Replaces the CUDA driver set-up in CUDAAllocator's constructor
 * (reference csrc/backend/cuda/allocator.cu:20-25). ormi_hip_init fails with
 * ORMI_HIP_ERR_NO_DEVICE when no GPU is visible, which makes the HIP device
 * absent the same way a throwing CUDAAllocator constructor does
 * (reference csrc/tests/test_utils.h:17-21). A device of another architecture
 * than the one the library was built for (gfx950, the target its kernels are
 * written and tuned for) is refused with ORMI_HIP_ERR_UNSUPPORTED. */
int ormi_hip_device_count(int* count);
int ormi_hip_init(int device);

typedef struct ormi_hip_props {
    char     name[64];         /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int      compute_units;    /* 256 on MI355X                              */
    int      clock_khz;
    int      lds_bytes_per_block;
    size_t   total_mem_bytes;
} ormi_hip_props;
int ormi_hip_get_props(ormi_hip_props* out);

/* Message for the last failing call on this thread ("" if none).
 * Replaces the exceptions thrown by CUDA_SAFE_CALL / NVRTC_SAFE_CALL
 * (reference csrc/utils/macros.h:8-19); the C++ side rethrows it as
 * std::runtime_error("HIP Error: ..."). */
const char* ormi_hip_last_error(void);

/* ---------------------------------------------------------------- memory --
 * Backs HIPAllocator : IAllocator (reference interface csrc/core/allocator.h:7-21,
 * CUDA implementation csrc/backend/cuda/allocator.cu:36-95). */
int ormi_hip_malloc(void** ptr, size_t bytes);                       /* cuMemAlloc   allocator.cu:47 */
int ormi_hip_free(void* ptr);                                        /* cuMemFree    allocator.cu:30 */
int ormi_hip_memset_d8(void* dst, unsigned char value, size_t count);/* cuMemsetD8   allocator.cu:58,81 */
int ormi_hip_memset_d32(void* dst, uint32_t value, size_t count);    /* cuMemsetD32  allocator.cu:76 */
/* Fill count elements of elem_bytes (1, 2, 4 or 8) with the pattern at value
 * (a small kernel, not hipMemset). fill_n for every dtype. */
int ormi_hip_fill(void* dst, const void* value, size_t elem_bytes, size_t count);
/* cuMemcpyHtoD allocator.cu:94, stream-ordered: src is copied into pinned
 * staging before the call returns (the caller may reuse it at once) and the
 * device copy runs after the work already on the stream, without blocking. */
int ormi_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int ormi_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);   /* cuMemcpyDtoH allocator.cu:90 */
int ormi_hip_memcpy_d2d(void* dst, const void* src, size_t bytes);   /* cuMemcpyDtoD allocator.cu:62 */
int ormi_hip_synchronize(void);

/* Contiguous element-type conversion dst[i] = (dst_dtype) src[i]. To a float
 * type it rounds to nearest even (int64 and int32 values past 2^24 included).
 * From a float type to an integer type it truncates toward zero, NaN gives 0
 * and out-of-range values saturate; to bool it is x != 0 (NaN gives true).
 * Between integer types (bool included) it is exact, an int64 outside the
 * int32 range saturating. */
int ormi_hip_convert(void* dst, int dst_dtype, const void* src, int src_dtype, size_t count);

/* ------------------------------------------------------------- hipRTC JIT --
 * Replaces compile_ptx + cuModuleLoadDataEx + cuModuleGetFunction + the
 * per-call cuModuleUnload (reference csrc/backend/cuda/utils.cu:6-27,
 * jit.cu:21-24,42-43). Compiles HIP source for the current device's gfx
 * target and caches the code object by (source, options, kernel name):
 * the same request returns the same handle without recompiling.
 * On ORMI_HIP_ERR_COMPILE, ormi_hip_last_error() holds the compiler log. */
int ormi_hip_rtc_compile(const char* source, const char* kernel_name,
                         const char* const* options, int num_options,
                         uint64_t* handle);

/* Same as ormi_hip_rtc_compile but only produces the code object (no module
 * load), so it runs without a GPU; target is a gfx name such as "gfx950".
 * Writes the code object size to *code_bytes. Used to check generated
 * source on a machine with no GPU. */
int ormi_hip_rtc_compile_only(const char* source, const char* target,
                              const char* const* options, int num_options,
                              size_t* code_bytes);

/* Launch a compiled kernel (reference cuLaunchKernel, jit.cu:40). args is the
 * kernelParams array: one pointer per kernel parameter. */
int ormi_hip_launch(uint64_t handle, const uint32_t grid[3], const uint32_t block[3],
                    uint32_t lds_bytes, void** args);

/* Queued launch of a compiled kernel whose parameters are all 8 bytes wide
 * (the generated kernels' convention): args holds num_args parameter values
 * (not pointers to them), copied before the call returns. The launch is issued
 * to the stream, after every earlier launch, by the library's launch thread,
 * so the calling thread does not pay the launch itself. Stream order is kept:
 * every other entry point that touches the device (copies, fills, GEMMs,
 * reductions, events, synchronize, free) first waits until all queued launches
 * are issued. An error of a queued launch is returned by the next such call.
 * Replaces cuLaunchKernel for generated kernels (reference jit.cu:40). */
#define ORMI_HIP_QUEUED_MAX_ARGS 128
int ormi_hip_launch_queued(uint64_t handle, const uint32_t grid[3], const uint32_t block[3],
                           uint32_t lds_bytes, const uint64_t* args, int num_args);

/* Number of distinct code objects compiled so far (cache misses). */
int ormi_hip_rtc_cache_size(uint64_t* entries);

/* ------------------------------------------------------------------ GEMM --
 * Replaces cuda::matmul's cublasSgemmBatched call and its per-call pointer
 * arrays (reference csrc/backend/cuda/kernels/blas/matmul.cu:19-112,
 * interface cuda_matmul.cuh:6-12). Row-major semantics of the reference:
 *   C[b][m][n] = sum_k A[b][m][k] * B[b][k][n]
 * A[m][k] lives at a + m*a_stride_m + k*a_stride_k (elements); normally one of
 * the two strides is 1 (stride_k == 1: "N", stride_m == 1: "T", the reference's
 * trans rule matmul.cu:47-52). Same for B with (stride_k, stride_n). Other
 * strides are accepted: for a large product such operands (and those whose
 * unit-stride extent or other strides are not whole 16-byte chunks) are first
 * copied into a zero-padded, k-contiguous device buffer the library keeps and
 * grows on demand; small products run a generic kernel.
 * C is written contiguous: C[b][m][n] at c + b*M*N + m*N + n, fp32.
 * dtype: ORMI_DTYPE_F32 (fp32 MFMA), ORMI_DTYPE_BF16 or ORMI_DTYPE_F16
 * (MFMA with fp32 accumulation). Batch index b decomposes row-major over
 * batch_shape[0..batch_ndim); each operand's batch offset is
 * sum(coord[i] * {a,b}_batch_stride[i]) — a stride of 0 broadcasts.
 * M == 0 or N == 0 is a no-op; K == 0 writes zeros to C and reads neither
 * operand (a and b may then be null). */
#define ORMI_GEMM_MAX_BATCH_DIMS 4
typedef struct ormi_gemm_desc {
    int         dtype;
    int         M, N, K;
    const void* a;
    int64_t     a_stride_m, a_stride_k;
    const void* b;
    int64_t     b_stride_k, b_stride_n;
    float*      c;
    int         batch_ndim;
    int         batch_shape[ORMI_GEMM_MAX_BATCH_DIMS];
    int64_t     a_batch_stride[ORMI_GEMM_MAX_BATCH_DIMS];
    int64_t     b_batch_stride[ORMI_GEMM_MAX_BATCH_DIMS];
} ormi_gemm_desc;
int ormi_hip_gemm(const ormi_gemm_desc* desc);

/* GEMM with an element-wise epilogue: each output element v = (A B)[b][m][n]
 * is transformed before it is stored, so a pointwise consumer of the product
 * needs no second pass over it. The reference's cublasSgemmBatched call fixes
 * alpha = 1, beta = 0 (matmul.cu:94-103); these kinds generalize that
 * C = alpha A B + beta C step to the consumers autograd and an SGD update put
 * on a matmul. Arithmetic is fp32 in exactly the order written below, with
 * no fused multiply-add, so the result matches the unfused element-wise
 * kernel bit for bit.
 *   ORMI_GEMM_EPI_NONE       C = v
 *   ORMI_GEMM_EPI_ADD        t = (s ? v * s[0] : v);
 *                            form 0: C = D + t   1: C = D - t   2: C = t - D
 *   ORMI_GEMM_EPI_UNARY      C = fn(v); aux (when not NULL) = v, laid out like C
 *   ORMI_GEMM_EPI_MUL_FN_D   C = v * fn(D)
 * D[b][m][n] is read at d + sum(coord[i] * d_batch_stride[i]) + m*d_stride_m
 * + n*d_stride_n (fp32; a stride of 0 broadcasts), s at s[0] (fp32, device
 * memory). fn is one of the ORMI_GEMM_FN_* functions, with the same device
 * code the fused element-wise kernels use. NULL epi is ORMI_GEMM_EPI_NONE.
 * C, aux and D must not overlap unless D == C with C's own layout (an
 * in-place update reads each element before writing it). */
enum {
    ORMI_GEMM_EPI_NONE = 0,
    ORMI_GEMM_EPI_ADD = 1,
    ORMI_GEMM_EPI_UNARY = 2,
    ORMI_GEMM_EPI_MUL_FN_D = 3
};
enum {
    ORMI_GEMM_FN_IDENTITY = 0,
    ORMI_GEMM_FN_RELU = 1,
    ORMI_GEMM_FN_STEP = 2,
    ORMI_GEMM_FN_TANH = 3,
    ORMI_GEMM_FN_TANH_GRAD = 4,
    ORMI_GEMM_FN_SIGMOID = 5,
    ORMI_GEMM_FN_SIGMOID_GRAD = 6,
    ORMI_GEMM_FN_GELU = 7,
    ORMI_GEMM_FN_GELU_GRAD = 8
};
typedef struct ormi_gemm_epilogue {
    int          kind;   /* ORMI_GEMM_EPI_* */
    int          fn;     /* ORMI_GEMM_FN_*: UNARY and MUL_FN_D */
    int          form;   /* ADD: 0, 1 or 2 */
    const float* s;      /* ADD: scale, or NULL for none */
    const float* d;      /* ADD and MUL_FN_D */
    int64_t      d_stride_m, d_stride_n;
    int64_t      d_batch_stride[ORMI_GEMM_MAX_BATCH_DIMS];
    float*       aux;    /* UNARY: also store v here, or NULL */
} ormi_gemm_epilogue;
int ormi_hip_gemm_ex(const ormi_gemm_desc* desc, const ormi_gemm_epilogue* epi);

/* ormi_hip_gemm_ex without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc). Same kernels, same results
 * bit for bit; the split-K partials and the finish pass's input live in a
 * static device array of ORMI_GEMM_NOALLOC_SCRATCH_BYTES that the library's
 * code object carries (held by each GPU until the process ends) instead of the
 * grown-on-demand workspace. A shape whose workspace (batch * M * N * splits *
 * 4 bytes, when the K split or the epilogue needs one) exceeds it returns
 * ORMI_HIP_ERR_INVALID and launches nothing. Like every entry point it
 * launches on the null stream, so it cannot be recorded into a HIP graph (the
 * null stream cannot be captured). All calls in a process share the array:
 * the library enqueues each call's kernels under one lock on that one stream,
 * so calls through this ABI never overlap. */
#define ORMI_GEMM_NOALLOC_SCRATCH_BYTES (32u << 20)
int ormi_hip_gemm_ex_noalloc(const ormi_gemm_desc* desc, const ormi_gemm_epilogue* epi);

/* Two products as one call: the result is that of ormi_hip_gemm_ex(d0, e0)
 * followed by ormi_hip_gemm_ex(d1, e1), bit for bit. Replaces the two
 * independent cuda::matmul calls (csrc/backend/cuda/kernels/blas/matmul.cu:
 * 19-122) the reference's MATMUL backward issues on one dZ: dX = dZ Y^T and
 * dY = X^T dZ (csrc/core/ops/blas/matmul.cpp:84-124), one after the other.
 * When neither product writes what the other reads or writes and each would
 * run alone as the fp32 128x128-tile kernel (one batch, M and N multiples of
 * 128, K of 32, at least one tile per compute unit, no K split, its epilogue
 * NONE or in the store), and their layouts and epilogues are the pair the
 * kernel is built for (one product with both operands k-contiguous, NONE or
 * MUL_FN_D, the other with both mn-contiguous, NONE or ADD: dZ W^T with the
 * activation's derivative and X^T dZ with the SGD update), both run as ONE
 * persistent launch whose work-groups take the first product's tiles, then the
 * second's, through one pipeline: the fill, the epilogue latency and the
 * last-wave tail are paid once instead of twice. That pays for shallow pairs
 * (2-6% at up to 64 k-tiles of 32 per work-group) and not for deep ones, so by
 * default only pairs of at most 64 k-tiles per work-group are grouped.
 * Otherwise the two run in order as their own calls would. *grouped
 * (if not NULL) is set to 1 when they ran as one launch, else 0. Both
 * descriptors are checked before anything is launched: an invalid one returns
 * its error and launches nothing. ORMI_GEMM_PAIR=0 turns grouping off, =2
 * groups every eligible pair whatever its depth. */
int ormi_hip_gemm_pair(const ormi_gemm_desc* d0, const ormi_gemm_epilogue* e0, const ormi_gemm_desc* d1,
                       const ormi_gemm_epilogue* e1, int* grouped);

/* ------------------------------------------------------------- reduction --
 * Replaces the reference's reduction kernel entry
 *   cuda::sum(in_buf, in_view, axes, out_view, keepdims)
 * (csrc/backend/cuda/kernels/reduce/cuda_sum.cuh:5-11, implemented with one
 * atomicAdd per element in sum.cu:12-97), and adds max and argmax. The library
 * generates, caches and launches the same hipRTC kernels the fusion scheduler
 * uses for a reduction with no element-wise prologue: a wave64 per row with
 * DPP reductions, LDS-combined column waves, and a second kernel that finishes
 * a split reduced range in part order (deterministic, no atomics).
 * The input is any strided view: x[i0..i(ndim-1)] at in + sum(i_d * strides[d])
 * elements (a stride of 0 broadcasts, negative strides are allowed). axes lists
 * the reduced dims (any order, no repeats); naxes == 0 reduces every dim.
 * out receives prod(kept extents) values, contiguous in the kept dims' order
 * (keepdims only changes the shape the caller puts on it): fp32 for SUM and
 * MAX (of the input converted to fp32), int64 indices for ARGMAX (row-major
 * position within the reduced dims, first occurrence; NaN counts as the
 * largest). An empty output is a no-op; SUM over an empty range writes 0; MAX
 * and ARGMAX over an empty range are ORMI_HIP_ERR_INVALID.
 * Workspace: a reduction split across work-groups needs
 * ormi_hip_reduce_workspace_size() bytes of device memory for its partials.
 * Pass it in workspace / workspace_bytes, or leave workspace NULL and the
 * library uses a buffer of its own (grown on demand, kept). */
#define ORMI_REDUCE_MAX_DIMS 8
enum { ORMI_REDUCE_SUM = 0, ORMI_REDUCE_MAX = 1, ORMI_REDUCE_ARGMAX = 2 };
typedef struct ormi_reduce_desc {
    int         op;                               /* ORMI_REDUCE_*                   */
    int         in_dtype;                         /* ORMI_DTYPE_* of the input        */
    const void* in;
    int         ndim;                             /* 0..ORMI_REDUCE_MAX_DIMS          */
    int         shape[ORMI_REDUCE_MAX_DIMS];
    int64_t     strides[ORMI_REDUCE_MAX_DIMS];    /* elements                         */
    int         naxes;
    int         axes[ORMI_REDUCE_MAX_DIMS];
    void*       out;
    void*       workspace;                        /* optional (NULL: library-owned)   */
    size_t      workspace_bytes;
} ormi_reduce_desc;
int ormi_hip_reduce_workspace_size(const ormi_reduce_desc* desc, size_t* bytes);
int ormi_hip_reduce(const ormi_reduce_desc* desc);

/* ------------------------------------------------------------------ map --
 * Replaces the reference's element-wise JIT entry cuda::execute_jit(root)
 * (csrc/backend/cuda/jit.cu:13-44) and the tape it compiles
 * (csrc/backend/cuda/compiler.cu:22-51: realized nodes become leaves, every
 * other node one instruction over earlier values). The caller passes that tape;
 * the library generates one gfx950 kernel for it (128-bit accesses, row-aligned
 * tiles, grid-stride over the compute units; the fusion scheduler's generator),
 * caches it by structure, and launches it on its stream.
 * Values: 0..num_leaves-1 are the leaves, num_leaves + k is insts[k]; an
 * instruction reads only earlier values. Arithmetic is fp32 whatever the leaf
 * dtypes (leaves are converted on load, as the reference computes in float).
 * Leaf strides are in elements and aligned to the map's shape (0 on a
 * broadcast dim, negative allowed); a scalar leaf reads its element 0 at every
 * position (the reference's 1-element rule, csrc/backend/cpu/jit.cpp:24).
 * Each output is a contiguous buffer of the map's shape holding one value,
 * stored as its dtype; several outputs make one kernel that evaluates the tape
 * once (multi-output fusion). Outputs must not overlap each other or a leaf.
 * Every leaf and output address is aligned to its element size.
 * An empty shape (a zero extent) is a no-op. Buffers may be released through
 * ormi_hip_free at once: it waits until the launch has been issued. */
#define ORMI_MAP_MAX_DIMS 8
#define ORMI_MAP_MAX_OUTPUTS 16
enum {
    ORMI_MAP_NEG = 0, ORMI_MAP_EXP = 1, ORMI_MAP_LOG = 2, ORMI_MAP_SIN = 3, ORMI_MAP_COS = 4,
    ORMI_MAP_ADD = 5, ORMI_MAP_SUB = 6, ORMI_MAP_MUL = 7, ORMI_MAP_DIV = 8, ORMI_MAP_POW = 9,
    ORMI_MAP_RELU = 10, ORMI_MAP_STEP = 11, ORMI_MAP_TANH = 12, ORMI_MAP_TANH_GRAD = 13,
    ORMI_MAP_SIGMOID = 14, ORMI_MAP_SIGMOID_GRAD = 15, ORMI_MAP_GELU = 16, ORMI_MAP_GELU_GRAD = 17,
    ORMI_MAP_EQ = 18,   /* 1.0f where a == b, else 0.0f */
    ORMI_MAP_CAST = 19  /* round to bf16 or f16 (f32: unchanged); integer results come from an output dtype */
};
typedef struct ormi_map_leaf {
    const void* ptr;
    int         dtype;                          /* ORMI_DTYPE_*                       */
    int         scalar;                         /* nonzero: element 0 everywhere      */
    int64_t     strides[ORMI_MAP_MAX_DIMS];     /* elements, aligned to shape         */
} ormi_map_leaf;
typedef struct ormi_map_inst {
    int op;                                     /* ORMI_MAP_*                         */
    int a, b;                                   /* operand values; b only for binary  */
    int dtype;                                  /* ORMI_MAP_CAST: ORMI_DTYPE_BF16/F16/F32 */
} ormi_map_inst;
typedef struct ormi_map_desc {
    int                  ndim;                  /* 0..ORMI_MAP_MAX_DIMS               */
    int                  shape[ORMI_MAP_MAX_DIMS];
    int                  num_leaves;
    const ormi_map_leaf* leaves;
    int                  num_insts;
    const ormi_map_inst* insts;
    int                  num_outputs;           /* 1..ORMI_MAP_MAX_OUTPUTS            */
    const int*           output_values;         /* value stored by each output        */
    void* const*         outputs;
    const int*           output_dtypes;         /* ORMI_DTYPE_*                       */
} ormi_map_desc;
int ormi_hip_map(const ormi_map_desc* desc);

/* ------------------------------------------------------ fused reduction --
 * ormi_hip_reduce over the values of an element-wise tape instead of a stored
 * input. Where the reference realizes the producer into a buffer and then
 * sums that buffer (csrc/backend/runtime.cpp:16-18 realizes every parent
 * first; cuda::sum, csrc/backend/cuda/kernels/reduce/cuda_sum.cuh:5-11), the
 * tape here runs as the reduction kernel's prologue and its values are never
 * stored: the fusion scheduler's reduction with a fused producer, for callers
 * that hold only this library. prologue is an ormi_map_desc whose shape is the
 * reduction's input shape; num_outputs must be 1 and output_values[0] names
 * the reduced value (its buffer and dtype fields are not read and may be
 * NULL). op, axes (over prologue->shape; naxes 0 = all), out and the
 * optional workspace are as in ormi_reduce_desc. */
typedef struct ormi_reduce_map_desc {
    const ormi_map_desc* prologue;
    int                  op;                       /* ORMI_REDUCE_*                    */
    int                  naxes;
    int                  axes[ORMI_REDUCE_MAX_DIMS];
    void*                out;
    void*                workspace;                /* optional (NULL: library-owned)   */
    size_t               workspace_bytes;
} ormi_reduce_map_desc;
int ormi_hip_reduce_map_workspace_size(const ormi_reduce_map_desc* desc, size_t* bytes);
int ormi_hip_reduce_map(const ormi_reduce_map_desc* desc);

/* ---------------------------------------------------------------- timing --
 * HIP events on the library's stream, for measuring kernel time from
 * outside (benchmarks). */
int ormi_hip_event_create(void** event);
int ormi_hip_event_record(void* event);
int ormi_hip_event_elapsed_ms(void* start, void* end, float* ms);
int ormi_hip_event_destroy(void* event);

#ifdef __cplusplus
}
#endif
#endif /* ORMI_HIP_H */
