"""The C-ABI from several host threads at once.

The header promises thread-safe memory entry points and launches issued in
call order on the one stream (the reference drives execution from one thread
and locks only its allocator, csrc/backend/cuda/allocator.cu:16,37,53). Here
four threads call ormi_hip_malloc / memcpy / fill / gemm_ex / free
concurrently (ctypes releases the GIL around each call). The GEMM shapes take
the K split and the epilogue's finish pass, so the threads share the library's
grown-on-demand workspace and its lock. Each thread checks its own results:
products within the fp32 accumulation bound 2 K eps32 (|A| |B|) of float64,
the SGD epilogue against the same bound, fills exactly.
"""
import ctypes
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class GemmDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int),
                ("a", ctypes.c_void_p), ("a_stride_m", ctypes.c_int64), ("a_stride_k", ctypes.c_int64),
                ("b", ctypes.c_void_p), ("b_stride_k", ctypes.c_int64), ("b_stride_n", ctypes.c_int64),
                ("c", ctypes.c_void_p), ("batch_ndim", ctypes.c_int), ("batch_shape", ctypes.c_int * 4),
                ("a_batch_stride", ctypes.c_int64 * 4), ("b_batch_stride", ctypes.c_int64 * 4)]


class GemmEpilogue(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("fn", ctypes.c_int), ("form", ctypes.c_int), ("s", ctypes.c_void_p),
                ("d", ctypes.c_void_p), ("d_stride_m", ctypes.c_int64), ("d_stride_n", ctypes.c_int64),
                ("d_batch_stride", ctypes.c_int64 * 4), ("aux", ctypes.c_void_p)]


# (M, N, K): few tiles and a deep K (a K split and its finish pass), whole
# tiles, ragged edges, and a depth that is not a multiple of the tile depth.
SHAPES = [(128, 128, 2048), (256, 512, 1024), (200, 136, 300), (64, 1024, 4096), (384, 384, 96)]


def worker(lib, tid, iters, errors):
    rng = np.random.default_rng(1000 + tid)
    held = []

    def put(a):
        a = np.ascontiguousarray(a, np.float32)
        p = ctypes.c_void_p()
        assert lib.ormi_hip_malloc(ctypes.byref(p), max(a.nbytes, 4)) == 0, lib.ormi_hip_last_error()
        assert lib.ormi_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes) == 0, lib.ormi_hip_last_error()
        held.append(p)
        return p

    def get(p, shape):
        out = np.empty(shape, np.float32)
        assert lib.ormi_hip_memcpy_d2h(out.ctypes.data, p, out.nbytes) == 0, lib.ormi_hip_last_error()
        return out

    try:
        for it in range(iters):
            M, N, K = SHAPES[(tid + it) % len(SHAPES)]
            A = (rng.standard_normal((M, K)) / 8).astype(np.float32)
            B = (rng.standard_normal((K, N)) / 8).astype(np.float32)
            W = rng.standard_normal((M, N)).astype(np.float32)
            g = GemmDesc(dtype=0, M=M, N=N, K=K, a=put(A), a_stride_m=K, a_stride_k=1, b=put(B), b_stride_k=N,
                         b_stride_n=1, c=put(W))
            lr = np.float32(0.5)
            e = GemmEpilogue(kind=1, form=1, s=put(np.array([lr], np.float32)), d=g.c, d_stride_m=N, d_stride_n=1)
            assert lib.ormi_hip_gemm_ex(ctypes.byref(g), ctypes.byref(e)) == 0, lib.ormi_hip_last_error()
            got = get(g.c, (M, N)).astype(np.float64)
            prod = A.astype(np.float64) @ B.astype(np.float64)
            bound = 2 * K * np.finfo(np.float32).eps * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
            want = W.astype(np.float64) - prod * float(lr)
            assert np.all(np.abs(got - want) <= bound * float(lr) + 2 * np.finfo(np.float32).eps * np.abs(want) + 1e-30), \
                (tid, it, M, N, K)
            # a plain product into a fresh buffer, then a fill over it
            c2 = put(np.zeros((M, N), np.float32))
            g.c = c2
            assert lib.ormi_hip_gemm_ex(ctypes.byref(g), None) == 0, lib.ormi_hip_last_error()
            assert np.all(np.abs(get(c2, (M, N)) - prod) <= bound + 1e-30), (tid, it)
            v = ctypes.c_float(float(tid) + 0.25)
            assert lib.ormi_hip_fill(c2, ctypes.byref(v), 4, M * N) == 0, lib.ormi_hip_last_error()
            assert np.all(get(c2, (M, N)) == np.float32(tid + 0.25))
            for p in held:
                assert lib.ormi_hip_free(p) == 0, lib.ormi_hip_last_error()
            held.clear()
    except BaseException as exc:  # reported by the main thread
        errors.append((tid, repr(exc)))
    finally:
        for p in held:
            lib.ormi_hip_free(p)


def test_four_threads_share_the_library(cabi, hip):
    # cabi is shared across modules: no argtypes are set (byref needs none)
    errors = []
    threads = [threading.Thread(target=worker, args=(cabi, t, 12, errors)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=240)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
    assert cabi.ormi_hip_synchronize() == 0
