"""ormi_hip_gemm_ex_noalloc: the allocation-free GEMM entry.

It runs the kernels of ormi_hip_gemm_ex with the split-K partials and the
finish pass's input in the library's static scratch array, so its results are
compared with ormi_hip_gemm_ex's bit for bit, on consecutive calls (the second
smaller, over the first call's leftover scratch contents), and a shape whose
workspace exceeds the array is refused without launching anything.
"""
import ctypes

import numpy as np
import pytest

from test_gemm_epilogue import Desc, Dev, Epi, bf16_bits, bits_equal

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # ORMI_GEMM_NOALLOC_SCRATCH_BYTES


def run_both(cabi, dev, dtype, M, K, N, epi_kind=0, seed=0, batch=1):
    """C from ormi_hip_gemm_ex and from the no-alloc entry on the same inputs."""
    rng = np.random.default_rng(seed)
    A = (rng.standard_normal((batch, M, K)) / 16).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    Dm = rng.standard_normal((batch, M, N)).astype(np.float32)
    s = np.array(0.25, np.float32)
    pa, pb = (dev.put(bf16_bits(A)), dev.put(bf16_bits(B))) if dtype == 3 else (dev.put(A), dev.put(B))
    pd, ps = dev.put(Dm), dev.put(s)
    outs = []
    for fn in (cabi.ormi_hip_gemm_ex, cabi.ormi_hip_gemm_ex_noalloc):
        pc = dev.put(np.full((batch, M, N), np.nan, np.float32))
        px = dev.put(np.full((batch, M, N), np.nan, np.float32))
        d = Desc(dtype=dtype, M=M, N=N, K=K, a=pa, a_stride_m=K, a_stride_k=1, b=pb, b_stride_k=N, b_stride_n=1, c=pc)
        if batch > 1:
            d.batch_ndim, d.batch_shape[0], d.a_batch_stride[0], d.b_batch_stride[0] = 1, batch, M * K, 0
        e = None
        if epi_kind == 1:    # C = D - (A B) s
            e = Epi(kind=1, fn=0, form=1, s=ps, d=pd, d_stride_m=N, d_stride_n=1)
            e.d_batch_stride[0] = M * N
        elif epi_kind == 2:  # C = gelu(A B), aux = A B
            e = Epi(kind=2, fn=7, aux=px)
        rc = fn(ctypes.byref(d), ctypes.byref(e) if e is not None else None)
        assert rc == 0, cabi.ormi_hip_last_error()
        outs.append((dev.get(pc, (batch, M, N)), dev.get(px, (batch, M, N)) if epi_kind == 2 else None))
    return outs


@pytest.mark.parametrize("calls", [
    # (dtype, M, K, N, epilogue kind, batch): the first call of each pair is the larger
    [(0, 256, 4096, 256, 0, 1), (0, 64, 2048, 128, 0, 1)],     # fp32, K split, plain store from the finish pass
    [(0, 128, 4096, 256, 2, 1), (0, 96, 1024, 64, 2, 1)],      # fp32 gelu + aux through the finish pass
    [(3, 512, 2048, 512, 1, 2), (3, 256, 512, 128, 1, 1)],     # bf16 (finish pass applies the epilogue), batched
    [(0, 256, 0, 256, 1, 1), (0, 32, 0, 16, 1, 1)],            # K = 0: zeros through the epilogue
])
def test_noalloc_matches_gemm_ex_twice(cabi, calls):
    dev = Dev(cabi)
    try:
        for i, (dtype, M, K, N, kind, batch) in enumerate(calls):
            (c_ref, x_ref), (c_got, x_got) = run_both(cabi, dev, dtype, M, K, N, kind, seed=90 + i, batch=batch)
            assert not np.isnan(c_ref).any()
            assert bits_equal(c_got, c_ref), (i, dtype, M, K, N)
            if kind == 2:
                assert bits_equal(x_got, x_ref)
    finally:
        dev.free()


def test_noalloc_refuses_oversized_workspace(cabi):
    """A bf16 4096 x 4096 product with an epilogue needs 64 MiB of workspace (the
    16-bit kernels apply epilogues in the finish pass): refused, C untouched."""
    M = N = 4096
    K = 64
    assert M * N * 4 > SCRATCH_BYTES
    dev = Dev(cabi)
    try:
        pa = dev.put(np.zeros((M, K), np.uint16))
        pb = dev.put(np.zeros((K, N), np.uint16))
        sentinel = np.full((M, N), 7.0, np.float32)
        pc, ps = dev.put(sentinel), dev.put(np.array(1.0, np.float32))
        d = Desc(dtype=3, M=M, N=N, K=K, a=pa, a_stride_m=K, a_stride_k=1, b=pb, b_stride_k=N, b_stride_n=1, c=pc)
        e = Epi(kind=1, fn=0, form=0, s=ps, d=pc, d_stride_m=N, d_stride_n=1)
        assert cabi.ormi_hip_gemm_ex_noalloc(ctypes.byref(d), ctypes.byref(e)) == 3
        assert b"allocation-free entry holds at most" in cabi.ormi_hip_last_error()
        assert np.array_equal(dev.get(pc, (M, N)), sentinel)
        # the allocating entry takes the same call
        assert cabi.ormi_hip_gemm_ex(ctypes.byref(d), ctypes.byref(e)) == 0, cabi.ormi_hip_last_error()
        assert np.array_equal(dev.get(pc, (M, N)), sentinel)  # 7 + 0 * 1
    finally:
        dev.free()
