"""The launch queue keeps stream order: generated kernels are issued by the
library's launch thread (ormi_hip_launch_queued), and every other device entry
point waits until the queue has issued what came before it."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def T(data, dev, **kw):
    from ormi_amd import Tensor

    return Tensor(data, dev, **kw)


def test_burst_of_queued_launches(hip):
    """2,000 realizes back to back (far more than one burst of the worker's
    spin), every result read afterwards."""
    x = np.arange(4096, dtype=np.float32)
    X = T(x, hip)
    outs = [(X + float(i)).realize() for i in range(2000)]
    for i in (0, 1, 777, 1999):
        assert np.array_equal(outs[i].numpy(), x + np.float32(i))


def test_upload_into_recycled_block_waits_for_queued_readers(hip):
    """A queued kernel reads a's buffer; a is dropped, its block returns to the
    pool, and the next upload of the same size reuses it. The upload must not
    overwrite the block before the queued reader has been issued."""
    rng = np.random.default_rng(81)
    for _ in range(50):
        a_np = rng.standard_normal(1 << 16).astype(np.float32)
        c_np = rng.standard_normal(1 << 16).astype(np.float32)
        a = T(a_np, hip)
        b = (a * 2.0 + 1.0).realize()
        del a
        c = T(c_np, hip)
        assert np.array_equal(b.numpy(), a_np * np.float32(2.0) + np.float32(1.0))
        assert np.array_equal(c.numpy(), c_np)


def test_gemm_reduction_and_events_after_queued_maps(hip, cabi):
    """A GEMM (launched by the calling thread) and a reduction read operands that
    queued maps produced; events bracket queued work."""
    rng = np.random.default_rng(82)
    a = rng.standard_normal((256, 128)).astype(np.float32)
    b = rng.standard_normal((128, 192)).astype(np.float32)
    A = T(a, hip)
    B = T(b, hip)
    A2 = (A * 0.5).realize()
    B2 = (B - 1.0).realize()
    got = (A2 @ B2).numpy()
    want = (a * np.float32(0.5)).astype(np.float64) @ (b - np.float32(1.0)).astype(np.float64)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4)
    s = ((A * 3.0).sum(1)).numpy()
    assert np.allclose(s, (a * np.float32(3.0)).astype(np.float64).sum(1), rtol=1e-5, atol=1e-4)
    cabi.ormi_hip_event_create.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    cabi.ormi_hip_event_record.argtypes = [ctypes.c_void_p]
    cabi.ormi_hip_event_elapsed_ms.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)]
    cabi.ormi_hip_event_destroy.argtypes = [ctypes.c_void_p]
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    assert cabi.ormi_hip_event_create(ctypes.byref(e0)) == 0 and cabi.ormi_hip_event_create(ctypes.byref(e1)) == 0
    big = T(np.ones((4096, 4096), np.float32), hip)
    assert cabi.ormi_hip_event_record(e0) == 0
    outs = [(big * float(i)).realize() for i in range(20)]
    assert cabi.ormi_hip_event_record(e1) == 0
    ms = ctypes.c_float()
    assert cabi.ormi_hip_event_elapsed_ms(e0, e1, ctypes.byref(ms)) == 0
    assert ms.value > 0.05  # 20 maps over 64 MB each ran between the two events
    assert outs[19].numpy()[123, 456] == 19.0
    cabi.ormi_hip_event_destroy(e0)
    cabi.ormi_hip_event_destroy(e1)


def test_queued_launch_rejects_bad_arguments(cabi, hip):
    grid = (ctypes.c_uint32 * 3)(1, 1, 1)
    block = (ctypes.c_uint32 * 3)(64, 1, 1)
    args = (ctypes.c_uint64 * 1)(0)
    cabi.ormi_hip_launch_queued.argtypes = [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint32),
                                            ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint32,
                                            ctypes.POINTER(ctypes.c_uint64), ctypes.c_int]
    assert cabi.ormi_hip_launch_queued(0, grid, block, 0, args, 1) == 3           # unknown handle
    assert cabi.ormi_hip_launch_queued(1, grid, block, 0, args, 129) == 3         # too many arguments
    assert b"ORMI_HIP_QUEUED_MAX_ARGS" in cabi.ormi_hip_last_error()
    assert cabi.ormi_hip_synchronize() == 0


def test_kernel_with_more_arguments_than_the_queue_holds(ob, hip):
    """A 130-leaf element-wise sum is one generated kernel with more than
    ORMI_HIP_QUEUED_MAX_ARGS (128) parameters: it takes the synchronous launch
    path, in order with the queued ones around it."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(83)
    arrs = [rng.integers(-8, 8, 256).astype(np.float32) for _ in range(130)]
    ts = [Tensor(a, hip) for a in arrs]
    before = (ts[0] * 2.0).realize()          # queued
    total = ts[0]
    for t in ts[1:]:
        total = total + t
    plan = ob._plan_kernel(total._node)
    assert plan["source"].count("const float* __restrict__ L") >= 128
    after = (total * 1.0).realize()           # the big kernel, then a queued map over it
    assert np.array_equal(after.numpy(), np.sum(arrs, axis=0, dtype=np.float32))
    assert np.array_equal(before.numpy(), arrs[0] * 2)


def test_failed_queued_launch_is_reported_not_lost(ob, cabi, hip):
    """A queued launch that failed (recorded through the library's test hook,
    as the launch thread records a launch the runtime refuses; no kernel runs)
    is reported by the next call that waits for the queue: empty_cache raises
    it after returning the cached blocks, and ormi_hip_free returns it after
    freeing its block. Each report clears it, so the call after succeeds."""
    cabi.ormi_hip_test_fail_queued_launch.argtypes = [ctypes.c_char_p]
    X = T(np.ones(1 << 16, np.float32), hip)
    del X  # one block in the cache
    assert ob.allocator_stats()["cached_bytes"] > 0
    assert cabi.ormi_hip_test_fail_queued_launch(b"refused") == 0
    with pytest.raises(RuntimeError, match="queued kernel launch: refused"):
        ob.empty_cache()
    assert ob.allocator_stats()["cached_bytes"] == 0
    assert cabi.ormi_hip_synchronize() == 0

    p = ctypes.c_void_p()
    assert cabi.ormi_hip_malloc(ctypes.byref(p), 1 << 20) == 0
    assert cabi.ormi_hip_test_fail_queued_launch(b"refused again") == 0
    assert cabi.ormi_hip_free(p) == 1  # ORMI_HIP_ERR_RUNTIME, after the hipFree
    assert b"queued kernel launch: refused again" in cabi.ormi_hip_last_error()
    assert cabi.ormi_hip_synchronize() == 0
    x = np.arange(1024, dtype=np.float32)
    assert np.array_equal((T(x, hip) * 2.0).numpy(), x * 2)
