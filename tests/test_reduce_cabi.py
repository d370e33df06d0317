"""ormi_hip_reduce through ctypes: the C-ABI reduction entry that replaces the
reference's cuda::sum(in_buf, in_view, axes, out_view, keepdims)
(csrc/backend/cuda/kernels/reduce/cuda_sum.cuh:5-11), with max and argmax.

GPU: row, column, global and multi-axis reductions over contiguous, transposed,
broadcast and bf16 inputs, against the CPU oracle (sum within the fp32 sum
bound; max and argmax bit-exact, ties to the first index, NaN first) and bit
for bit against the HIP core's own reductions (the same generated kernels);
caller-provided and library-owned workspaces; empty inputs.
CPU: descriptor validation (no compute).
"""
import ctypes
import zlib

import numpy as np
import pytest

from conftest import fp32_sum_tolerance

MAXD = 8
SUM, MAX, ARGMAX = 0, 1, 2
F32, BF16 = 0, 3


class ReduceDesc(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int), ("in_dtype", ctypes.c_int), ("in_", ctypes.c_void_p), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_int * MAXD), ("strides", ctypes.c_int64 * MAXD), ("naxes", ctypes.c_int),
                ("axes", ctypes.c_int * MAXD), ("out", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_size_t)]


def desc(op, dtype, ptr, shape, strides, axes, out, ws=None, ws_bytes=0):
    d = ReduceDesc(op=op, in_dtype=dtype, in_=ptr, ndim=len(shape), naxes=len(axes), out=out, workspace=ws,
                   workspace_bytes=ws_bytes)
    for i, (e, s) in enumerate(zip(shape, strides)):
        d.shape[i], d.strides[i] = e, s
    for i, a in enumerate(axes):
        d.axes[i] = a
    return d


# ------------------------------------------------------------------ CPU side
@pytest.mark.parametrize("fields,msg", [
    (dict(op=7), b"op must be"),
    (dict(in_dtype=9), b"unknown input dtype"),
    (dict(ndim=9), b"ndim must be"),
    (dict(naxes=3), b"naxes must be"),
    (dict(axes=(2,)), b"axis out of range"),
    (dict(axes=(1, 1)), b"repeated axis"),
    (dict(shape=(4, -1)), b"negative extent"),
    (dict(shape=(1 << 30, 1 << 30, 1 << 30)), b"more than 2^62 elements"),
    (dict(in_=0x1002), b"input is not aligned to its element size"),
    (dict(in_dtype=BF16, in_=0x1001), b"input is not aligned to its element size"),
    (dict(out=0x2002), b"output is not aligned to its element size"),
    (dict(op=ARGMAX, out=0x2004), b"output is not aligned to its element size"),  # int64 indices
    (dict(ws=0x3002), b"workspace is not 4-byte aligned"),
])
def test_reduce_descriptor_validation(cabi, fields, msg):
    base = dict(op=SUM, in_dtype=F32, shape=(4, 6), axes=(1,), in_=0x1000, out=0x2000, ws=None)
    base.update(fields)
    shape = base["shape"]
    d = desc(base["op"], base["in_dtype"], base["in_"], shape, [6] * (len(shape) - 1) + [1], base["axes"], base["out"],
             base["ws"], 1 << 20 if base["ws"] else 0)
    if "ndim" in fields:
        d.ndim = fields["ndim"]
    if "naxes" in fields:
        d.naxes = fields["naxes"]
    assert cabi.ormi_hip_reduce(ctypes.byref(d)) == 3
    assert msg in cabi.ormi_hip_last_error()
    assert cabi.ormi_hip_reduce(None) == 3


def test_reduce_empty_output_is_a_no_op(cabi):
    d = desc(MAX, F32, None, (0, 5), (5, 1), (1,), None)
    assert cabi.ormi_hip_reduce(ctypes.byref(d)) == 0
    size = ctypes.c_size_t(7)
    assert cabi.ormi_hip_reduce_workspace_size(ctypes.byref(d), ctypes.byref(size)) == 0 and size.value == 0


# ------------------------------------------------------------------ GPU side
class Dev:
    def __init__(self, lib):
        self.lib, self.ptrs = lib, []

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = ctypes.c_void_p()
        assert self.lib.ormi_hip_malloc(ctypes.byref(p), max(arr.nbytes, 4)) == 0
        if arr.nbytes:
            assert self.lib.ormi_hip_memcpy_h2d(p, arr.ctypes.data, arr.nbytes) == 0
        self.ptrs.append(p)
        return p

    def empty(self, nbytes):
        p = ctypes.c_void_p()
        assert self.lib.ormi_hip_malloc(ctypes.byref(p), max(nbytes, 4)) == 0
        self.ptrs.append(p)
        return p

    def get(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        assert self.lib.ormi_hip_synchronize() == 0
        if out.nbytes:
            assert self.lib.ormi_hip_memcpy_d2h(out.ctypes.data, p, out.nbytes) == 0
        return out

    def free(self):
        for p in self.ptrs:
            self.lib.ormi_hip_free(p)


def reduce_cabi(cabi, dev, op, x_view, base, base_ptr, strides_el, axes, dtype=F32, own_ws=False):
    """Reduce the view x_view (a numpy view of base, uploaded at base_ptr) with the C ABI."""
    shape = x_view.shape
    kept = [e for i, e in enumerate(shape) if i not in (axes or range(len(shape)))]
    out_np = np.int64 if op == ARGMAX else np.float32
    n_out = int(np.prod(kept)) if kept else 1
    out = dev.empty(n_out * np.dtype(out_np).itemsize)
    d = desc(op, dtype, base_ptr, shape, strides_el, axes, out)
    size = ctypes.c_size_t(0)
    assert cabi.ormi_hip_reduce_workspace_size(ctypes.byref(d), ctypes.byref(size)) == 0, cabi.ormi_hip_last_error()
    if own_ws and size.value:
        d.workspace, d.workspace_bytes = dev.empty(size.value), size.value
    assert cabi.ormi_hip_reduce(ctypes.byref(d)) == 0, cabi.ormi_hip_last_error()
    return dev.get(out, tuple(kept), out_np), size.value


def bits(a):
    return np.ascontiguousarray(a).reshape(-1).view(np.uint8)


def graph_reduce(x, op, axes, dev):
    """The same reduction through the Tensor API on dev (the oracle or the HIP core)."""
    from ormi_amd import Tensor

    t = Tensor(np.ascontiguousarray(x), dev)
    ax = tuple(axes) if axes else None
    return {SUM: t.sum, MAX: t.max, ARGMAX: t.argmax}[op](ax).numpy()


CASES = [
    # name, shape, axes
    ("row", (1024, 8192), (1,)),
    ("row_shared", (4103, 4108), (1,)),   # four waves per row, work-group cap
    ("row_few_rows", (3, 100003), (1,)),
    ("col", (4096, 2048), (0,)),
    ("col_ragged", (777, 131), (0,)),
    ("global", (1000003,), ()),
    ("axes02", (6, 40, 70), (0, 2)),
    ("middle", (5, 300, 9), (1,)),
    ("all_of_3d", (4, 5, 6), ()),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,shape,axes", CASES)
@pytest.mark.parametrize("op", [SUM, MAX, ARGMAX])
def test_reduce_cabi_vs_oracle_and_core(cabi, cpu, hip, name, shape, axes, op):
    from ormi_amd import Tensor

    rng = np.random.default_rng(zlib.crc32(f"{name}/{op}".encode()))
    x = rng.integers(-50, 50, shape).astype(np.float32) if op != SUM else rng.standard_normal(shape).astype(np.float32)
    dev = Dev(cabi)
    try:
        ptr = dev.put(x)
        strides = [s // 4 for s in x.strides]
        got, ws = reduce_cabi(cabi, dev, op, x, x, ptr, strides, list(axes))
        if op == ARGMAX and len(axes) > 1:
            # the graph API takes one axis (numpy's rule); the C ABI indexes the
            # reduced dims row-major, which numpy gives after moving them last
            kept = [i for i in range(x.ndim) if i not in axes]
            moved = np.moveaxis(x, list(axes), list(range(len(kept), x.ndim)))
            want = np.argmax(moved.reshape([x.shape[i] for i in kept] + [-1]), axis=-1)
        else:
            want = graph_reduce(x, op, axes, cpu)
            core = graph_reduce(x, op, axes, hip)   # the HIP core on the same input: same kernels
            assert got.dtype == core.dtype and np.array_equal(bits(got), bits(core))
        if op == SUM:
            exact = x.astype(np.float64).sum(axis=tuple(axes) if axes else None)
            assert np.all(np.abs(got - exact) <= fp32_sum_tolerance(x, tuple(axes) if axes else None))
            assert np.all(np.abs(got - want) <= 2 * fp32_sum_tolerance(x, tuple(axes) if axes else None))
        else:
            assert np.array_equal(got, want)
        if name in ("row_few_rows", "global"):
            assert ws > 0  # split reduced range: two passes through the workspace
            got2, _ = reduce_cabi(cabi, dev, op, x, x, ptr, strides, list(axes), own_ws=True)
            assert np.array_equal(bits(got2), bits(got))
    finally:
        dev.free()


@pytest.mark.gpu
def test_reduce_cabi_views_and_bf16(cabi, cpu, hip):
    """Transposed and broadcast (stride 0) views, negative strides, a bf16 input,
    ties and NaN for argmax."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(61)
    base = rng.integers(-4, 4, (300, 500)).astype(np.float32)
    base[17, 33] = np.nan
    dev = Dev(cabi)
    try:
        ptr = dev.put(base)
        # transposed view (500, 300): strides (1, 500)
        xt = base.T
        for op in (SUM, MAX, ARGMAX):
            got, _ = reduce_cabi(cabi, dev, op, xt, base, ptr, [1, 500], [1])
            want = graph_reduce(xt, op, (1,), cpu)
            if op == SUM:
                assert np.array_equal(np.isnan(got), np.isnan(want))
                m = ~np.isnan(want)
                assert np.array_equal(got[m], want[m])  # small integers: exact in any order
            else:
                assert np.array_equal(got, want, equal_nan=True)
        # broadcast: a (500,) row vector viewed as (64, 500) with stride 0 on dim 0
        row = base[5]
        got, _ = reduce_cabi(cabi, dev, SUM, np.broadcast_to(row, (64, 500)), base, ctypes.c_void_p(ptr.value + 5 * 500 * 4),
                             [0, 1], [0])
        assert np.array_equal(got, (row * 64).astype(np.float32))
        # negative stride: the last row read backwards
        rev = base[299, ::-1]
        last = ctypes.c_void_p(ptr.value + (299 * 500 + 499) * 4)
        got, _ = reduce_cabi(cabi, dev, ARGMAX, rev, base, last, [-1], [0])
        assert got.tolist() == int(np.argmax(rev))
        # bf16 input (exact small integers)
        bits = (base.view(np.uint32) >> 16).astype(np.uint16)
        pb = dev.put(bits)
        got, _ = reduce_cabi(cabi, dev, MAX, base, base, pb, [500, 1], [1], dtype=BF16)
        assert np.array_equal(got, Tensor(base, cpu, dtype="bfloat16").max(1).numpy(), equal_nan=True)
    finally:
        dev.free()


@pytest.mark.gpu
def test_reduce_cabi_empty_ranges(cabi, hip):
    dev = Dev(cabi)
    try:
        out = dev.put(np.full(5, 9.0, np.float32))
        d = desc(SUM, F32, None, (0, 5), (5, 1), (0,), out)
        assert cabi.ormi_hip_reduce(ctypes.byref(d)) == 0
        assert dev.get(out, (5,), np.float32).tolist() == [0.0] * 5
        d = desc(ARGMAX, F32, None, (0, 5), (5, 1), (0,), out)
        assert cabi.ormi_hip_reduce(ctypes.byref(d)) == 3
        assert b"no identity" in cabi.ormi_hip_last_error()
    finally:
        dev.free()
