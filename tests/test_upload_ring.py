"""Host-to-device copies are stream-ordered (ormi_hip_memcpy_h2d stages the
bytes in a 64 MiB pinned ring and enqueues an asynchronous copy), where the
reference's cuMemcpyHtoD blocks (csrc/backend/cuda/allocator.cu:61-67). These
check what the caller can observe: every byte arrives, in stream order with
kernels before and after, the caller's buffer may be reused on return, and an
upload does not wait for queued kernels to finish."""
import ctypes
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MiB = 1 << 20


def raw_roundtrip(cabi, data: bytes) -> bytes:
    n = len(data)
    p = ctypes.c_void_p()
    assert cabi.ormi_hip_malloc(ctypes.byref(p), max(n, 1)) == 0, cabi.ormi_hip_last_error()
    try:
        src = ctypes.create_string_buffer(data, n)
        assert cabi.ormi_hip_memcpy_h2d(p, src, n) == 0, cabi.ormi_hip_last_error()
        out = ctypes.create_string_buffer(n)
        assert cabi.ormi_hip_memcpy_d2h(out, p, n) == 0, cabi.ormi_hip_last_error()
        return out.raw
    finally:
        cabi.ormi_hip_free(p)


@pytest.mark.parametrize("n", [1, 3, 255, 256, 257, MiB + 3, 16 * MiB, 16 * MiB + 4, 40 * MiB + 12, 70 * MiB + 1])
def test_upload_sizes_across_pieces_and_wraps(cabi, hip, n):
    """Odd byte counts, exactly one 16 MiB piece, several pieces, and an upload
    larger than the 64 MiB ring (its pieces wrap over ones still in flight)."""
    rng = np.random.default_rng(n)
    data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
    assert raw_roundtrip(cabi, data) == data


def test_many_small_uploads_keep_their_bytes(hip):
    """6,000 uploads kept alive (more than the 4,096 pieces the ring tracks at
    once), with 1 MiB ones mixed in so the ring wraps several times, read back
    only at the end."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(91)
    arrs, ts = [], []
    for i in range(6000):
        n = 262144 if i % 500 == 0 else int(rng.integers(1, 3000))
        a = rng.standard_normal(n).astype(np.float32)
        arrs.append(a)
        ts.append(Tensor(a, hip))
    for a, t in zip(arrs, ts):
        assert np.array_equal(t.numpy(), a)


def test_caller_buffer_is_free_on_return(hip):
    """The bytes are copied out before the call returns: overwriting the source
    right after the upload (while the DMA may still be queued) changes nothing."""
    from ormi_amd import Tensor

    a = np.arange(3 * MiB, dtype=np.float32)
    keep = a.copy()
    t = Tensor(a, hip)
    a[:] = -1.0
    assert np.array_equal(t.numpy(), keep)


def test_upload_is_stream_ordered_with_kernels(hip):
    """A kernel reads an upload made right before it, and an upload into a block
    freed after a queued reader lands after that reader."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(92)
    for _ in range(30):
        x = rng.standard_normal(1 << 18).astype(np.float32)
        X = Tensor(x, hip)
        y = (X * 3.0 + 1.0).realize()
        del X
        z = rng.standard_normal(1 << 18).astype(np.float32)
        Z = Tensor(z, hip)  # may reuse X's block
        assert np.array_equal(y.numpy(), x * np.float32(3.0) + np.float32(1.0))
        assert np.array_equal(Z.numpy(), z)


def test_upload_does_not_wait_for_queued_kernels(hip):
    """Eight fp32 4096^3 products (about 1 ms each) are on the stream; a 4 KiB
    upload made behind them returns long before they finish. A synchronous copy
    would wait for all of them."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(93)
    a = (rng.standard_normal((4096, 4096)) / 64).astype(np.float32)
    A = Tensor(a, hip)
    (A @ A).numpy()  # warm up: kernel choice, allocator pool
    t0 = time.perf_counter()
    outs = [(A @ A).realize() for _ in range(8)]
    t1 = time.perf_counter()
    small = np.arange(1024, dtype=np.float32)
    S = Tensor(small, hip)
    t2 = time.perf_counter()
    last = outs[-1].numpy()
    t3 = time.perf_counter()
    chain = t3 - t0
    assert chain > 4e-3, f"the queued products took only {chain * 1e3:.2f} ms"
    assert t2 - t1 < chain / 4, f"upload took {(t2 - t1) * 1e3:.2f} ms behind {chain * 1e3:.2f} ms of kernels"
    assert np.array_equal(S.numpy(), small)
    ref = a[:64].astype(np.float64) @ a.astype(np.float64)
    assert np.allclose(last[:64], ref, rtol=1e-4, atol=1e-4)
