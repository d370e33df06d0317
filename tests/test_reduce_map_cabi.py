"""ormi_hip_reduce_map through ctypes: ormi_hip_reduce over a caller's
element-wise tape (an ormi_hip_map descriptor), evaluated as the reduction
kernel's prologue. It stands where the reference realizes the producer into a
buffer and then sums that buffer (csrc/backend/runtime.cpp:16-18, then
cuda::sum, csrc/backend/cuda/kernels/reduce/cuda_sum.cuh:5-11).

GPU: a tape and reduction through the C ABI give the graph path's bits (a
reduction whose element-wise input is unrealized fuses it as the same
prologue, through the same code generator), and match the CPU oracle: sums
within the fp32 sum bound of the tape's values (n eps32 sum|v|), max and argmax
exactly. Cases: the C1 forward (relu(a*b + c) * 0.5 summed over each row), a
column sum and a global sum of a broadcast-bias map, max and argmax of a scaled
and shifted input, a bf16 leaf, a two-pass reduction with the caller's
workspace and with the library's, empty inputs, and 24 random tapes (every op,
broadcast / transposed / scalar / 16-bit leaves) under random reductions,
bit for bit against the graph path.
CPU: descriptor validation (no compute)."""
import ctypes

import numpy as np
import pytest

from conftest import fp32_sum_tolerance
from test_map_cabi import Desc, make_desc
from test_reduce_cabi import Dev, bits

MAXD = 8
SUM, MAX, ARGMAX = 0, 1, 2
F32, BF16 = 0, 3


class ReduceMapDesc(ctypes.Structure):
    _fields_ = [("prologue", ctypes.POINTER(Desc)), ("op", ctypes.c_int), ("naxes", ctypes.c_int),
                ("axes", ctypes.c_int * MAXD), ("out", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_size_t)]


def rdesc(prologue, op, axes, out, ws=None, ws_bytes=0):
    d = ReduceMapDesc(prologue=ctypes.pointer(prologue) if prologue is not None else None, op=op, naxes=len(axes),
                      out=out, workspace=ws, workspace_bytes=ws_bytes)
    for i, a in enumerate(axes):
        d.axes[i] = a
    return d


@pytest.fixture(scope="module")
def lib(cabi):
    cabi.ormi_hip_reduce_map.argtypes = [ctypes.POINTER(ReduceMapDesc)]
    cabi.ormi_hip_reduce_map_workspace_size.argtypes = [ctypes.POINTER(ReduceMapDesc), ctypes.POINTER(ctypes.c_size_t)]
    return cabi


# ----------------------------------------------------------------- no GPU --
@pytest.mark.parametrize("case,msg", [
    (dict(op=5), b"op must be"),
    (dict(no_prologue=True), b"null prologue"),
    (dict(num_outputs=2), b"exactly one output value"),
    (dict(axes=(2,)), b"axis out of range"),
    (dict(axes=(0, 0)), b"repeated axis"),
    (dict(leaf_dtype=9), b"ormi_hip_reduce_map: leaf 0 has an unknown dtype"),
    (dict(a=3), b"ormi_hip_reduce_map: instruction 0: operand a must be an earlier value"),
    (dict(value=9), b"output 0 names no value"),
    (dict(out=None), b"null output"),
    (dict(out=0x2002), b"output is not aligned to its element size"),
    (dict(op=ARGMAX, out=0x2004), b"output is not aligned to its element size"),  # int64 indices
])
def test_reduce_map_rejects_bad_descriptors(lib, case, msg):
    pro, keep = make_desc((4, 8), [(0x1000, case.get("leaf_dtype", F32), False, (8, 1))],
                          [("EXP", case.get("a", 0), 0, F32)], [(case.get("value", 1), None, F32)])
    if "num_outputs" in case:
        pro.num_outputs = case["num_outputs"]
    d = rdesc(None if case.get("no_prologue") else pro, case.get("op", SUM), case.get("axes", (1,)),
              case.get("out", 0x2000))
    assert lib.ormi_hip_reduce_map(ctypes.byref(d)) == 3  # ORMI_HIP_ERR_INVALID
    assert msg in lib.ormi_hip_last_error()
    size = ctypes.c_size_t(5)
    assert lib.ormi_hip_reduce_map_workspace_size(ctypes.byref(d), ctypes.byref(size)) == 3 and size.value == 0
    assert lib.ormi_hip_reduce_map(None) == 3


def test_reduce_map_of_an_empty_output_is_a_no_op(lib):
    pro, keep = make_desc((0, 8), [(0x1000, F32, False, (8, 1))], [("EXP", 0, 0, F32)], [(1, None, F32)])
    d = rdesc(pro, MAX, (1,), None)
    assert lib.ormi_hip_reduce_map(ctypes.byref(d)) == 0


# -------------------------------------------------------------------- GPU --
def run(lib, dev, shape, leaves, insts, value, op, axes, own_ws=False):
    """The tape's value `value` reduced by op over axes with the C ABI; leaves:
    (device ptr, dtype, scalar, element strides)."""
    pro, keep = make_desc(shape, leaves, insts, [(value, None, F32)])
    kept = [e for i, e in enumerate(shape) if axes and i not in axes]
    out_np = np.int64 if op == ARGMAX else np.float32
    out = dev.empty(int(np.prod(kept)) * np.dtype(out_np).itemsize if kept else 8)
    d = rdesc(pro, op, axes, out)
    size = ctypes.c_size_t(0)
    assert lib.ormi_hip_reduce_map_workspace_size(ctypes.byref(d), ctypes.byref(size)) == 0, lib.ormi_hip_last_error()
    if own_ws and size.value:
        d.workspace, d.workspace_bytes = dev.empty(size.value), size.value
    assert lib.ormi_hip_reduce_map(ctypes.byref(d)) == 0, lib.ormi_hip_last_error()
    return dev.get(out, tuple(kept), out_np), size.value


def strides_of(a):
    return tuple(s // a.itemsize for s in a.strides)


@pytest.mark.gpu
def test_c1_forward_through_the_fused_reduction(lib, cpu, hip):
    """sum(relu(a*b + c) * 0.5, axis=1) over (1024, 1024), seed 0 as the C1
    config: the graph path's bits, the oracle within the fp32 sum bound."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(0)
    a, b, c = (rng.uniform(-1, 1, (1024, 1024)).astype(np.float32) for _ in range(3))
    half = np.array(0.5, np.float32)
    dev = Dev(lib)
    try:
        pa, pb, pc, ph = dev.put(a), dev.put(b), dev.put(c), dev.put(half)
        leaves = [(pa.value, F32, False, (1024, 1)), (pb.value, F32, False, (1024, 1)),
                  (pc.value, F32, False, (1024, 1)), (ph.value, F32, True, (0, 0))]
        insts = [("MUL", 0, 1, F32), ("ADD", 4, 2, F32), ("RELU", 5, -1, F32), ("MUL", 6, 3, F32)]
        got, _ = run(lib, dev, (1024, 1024), leaves, insts, 7, SUM, (1,))
        core = ((Tensor(a, hip) * Tensor(b, hip) + Tensor(c, hip)).relu() * 0.5).sum(1).numpy()
        assert np.array_equal(bits(got), bits(core))
        want = ((Tensor(a, cpu) * Tensor(b, cpu) + Tensor(c, cpu)).relu() * 0.5).sum(1).numpy()
        v = np.maximum(a * b + c, np.float32(0)) * half  # the tape's fp32 values, op by op
        bound = fp32_sum_tolerance(v, 1)
        assert np.all(np.abs(got - v.astype(np.float64).sum(1)) <= bound)
        assert np.all(np.abs(got - want) <= 2 * bound)
    finally:
        dev.free()


@pytest.mark.gpu
@pytest.mark.parametrize("axes", [(0,), ()])
def test_column_and_global_sums_of_a_broadcast_map(lib, cpu, hip, axes):
    """sum((x + bias) * s) with a bias row broadcast down the columns and a
    scalar s: a column sum (two passes over 4096 rows) and a global sum."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(71 + len(axes))
    x = rng.standard_normal((4096, 1536)).astype(np.float32)
    bias = rng.standard_normal(1536).astype(np.float32)
    s = np.array(0.75, np.float32)
    dev = Dev(lib)
    try:
        px, pbias, ps = dev.put(x), dev.put(bias), dev.put(s)
        leaves = [(px.value, F32, False, (1536, 1)), (pbias.value, F32, False, (0, 1)), (ps.value, F32, True, (0, 0))]
        insts = [("ADD", 0, 1, F32), ("MUL", 3, 2, F32)]
        got, ws = run(lib, dev, x.shape, leaves, insts, 4, SUM, axes)
        got_own, _ = run(lib, dev, x.shape, leaves, insts, 4, SUM, axes, own_ws=True)
        assert np.array_equal(bits(got), bits(got_own))
        ax = axes[0] if axes else None
        core = ((Tensor(x, hip) + Tensor(bias, hip)) * 0.75).sum(ax).numpy()
        assert np.array_equal(bits(got), bits(core))
        v = (x + bias) * s
        bound = fp32_sum_tolerance(v, ax)
        assert np.all(np.abs(got - v.astype(np.float64).sum(axis=ax)) <= bound)
        want = ((Tensor(x, cpu) + Tensor(bias, cpu)) * 0.75).sum(ax).numpy()
        assert np.all(np.abs(got - want) <= 2 * bound)
    finally:
        dev.free()


@pytest.mark.gpu
@pytest.mark.parametrize("op", [MAX, ARGMAX])
def test_max_and_argmax_of_a_scaled_shifted_input(lib, cpu, hip, op):
    """max / argmax over rows of x * s - t (t a per-row column (R, 1)), on a
    transposed x and with ties: exact against numpy and the oracle; the few-row
    case (3 rows of 100003) takes two passes, once with the caller's workspace,
    and 4100 rows of 1100 are shared by four waves each (strided, scalar loads)."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(83 + op)
    for rows, cols in ((2048, 1000), (3, 100003), (4100, 1100)):
        base = rng.integers(-20, 20, (cols, rows)).astype(np.float32)   # stored transposed
        x = base.T                                                     # (rows, cols), strides (1, rows)
        t = rng.integers(-3, 3, (rows, 1)).astype(np.float32)
        s = np.array(2.0, np.float32)
        dev = Dev(lib)
        try:
            px, pt, ps = dev.put(base), dev.put(t), dev.put(s)
            leaves = [(px.value, F32, False, (1, rows)), (ps.value, F32, True, (0, 0)), (pt.value, F32, False, (1, 0))]
            insts = [("MUL", 0, 1, F32), ("SUB", 3, 2, F32)]
            got, ws = run(lib, dev, (rows, cols), leaves, insts, 4, op, (1,))
            v = x * s - t
            want = v.max(1) if op == MAX else v.argmax(1)
            assert np.array_equal(got, want)
            X = Tensor(np.ascontiguousarray(x), cpu) * 2.0 - Tensor(t, cpu)
            assert np.array_equal(got, (X.max(1) if op == MAX else X.argmax(1)).numpy())
            if rows == 3:
                assert ws > 0
                got2, _ = run(lib, dev, (rows, cols), leaves, insts, 4, op, (1,), own_ws=True)
                assert np.array_equal(got2, got)
        finally:
            dev.free()


@pytest.mark.gpu
def test_bf16_leaf_in_the_prologue(lib, cpu, hip):
    """sum(x * 2 + c) over rows with x stored as bf16 (small integers, exact in
    any order) and c fp32: the oracle's values exactly."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(97)
    x = rng.integers(-8, 8, (512, 777)).astype(np.float32)
    c = rng.integers(-4, 4, (512, 777)).astype(np.float32)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    two = np.array(2.0, np.float32)
    dev = Dev(lib)
    try:
        px, pc, p2 = dev.put(xb), dev.put(c), dev.put(two)
        leaves = [(px.value, BF16, False, (777, 1)), (p2.value, F32, True, (0, 0)), (pc.value, F32, False, (777, 1))]
        insts = [("MUL", 0, 1, F32), ("ADD", 3, 2, F32)]
        got, _ = run(lib, dev, x.shape, leaves, insts, 4, SUM, (1,))
        want = (Tensor(x, cpu, dtype="bfloat16") * 2.0 + Tensor(c, cpu)).sum(1).numpy()
        assert np.array_equal(got, want)
        assert np.array_equal(got, (x * 2 + c).sum(1))
    finally:
        dev.free()


@pytest.mark.gpu
def test_reduce_map_empty_inputs(lib, hip):
    dev = Dev(lib)
    try:
        out = dev.put(np.full(5, 9.0, np.float32))
        pro, keep = make_desc((0, 5), [(None, F32, False, (5, 1))], [("EXP", 0, -1, F32)], [(1, None, F32)])
        d = rdesc(pro, SUM, (0,), out)
        assert lib.ormi_hip_reduce_map(ctypes.byref(d)) == 0
        assert dev.get(out, (5,), np.float32).tolist() == [0.0] * 5
        d = rdesc(pro, ARGMAX, (0,), out)
        assert lib.ormi_hip_reduce_map(ctypes.byref(d)) == 3
        assert b"no identity" in lib.ormi_hip_last_error()
    finally:
        dev.free()


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(24))
def test_random_tapes_reduce_as_the_graph_path(ob, lib, hip, seed):
    """Random tapes (every op, broadcast / transposed / scalar / 16-bit leaves,
    the generator of test_map_cabi) plus a full-shape leaf added to the last
    value, reduced by a random op over random axes: the C-ABI result equals
    the graph path's (a reduction of the same unrealized region) bit for bit,
    NaN and infinities included."""
    from ormi_amd import Tensor
    from test_map_cabi import BINARY, DT_NAME, random_case

    rng = np.random.default_rng(1000 + seed)
    shape, leaves, insts, _ = random_case(seed)
    nl = len(leaves)
    full = rng.uniform(-2, 2, shape).astype(np.float32)
    leaves = leaves + [dict(kind="plain", dtype=F32, data=full)]
    bump = lambda v: v + 1 if v >= nl else v  # instruction values move up past the new leaf
    insts = [(name, bump(a), bump(b) if b >= 0 else b, dt) for name, a, b, dt in insts]
    last = nl + len(insts)                    # the old last value, renumbered
    insts.append(("ADD", last, nl, F32))
    value = nl + len(insts)
    op = int(rng.integers(0, 3))
    nd = len(shape)
    if op == ARGMAX:
        axes = [int(rng.integers(0, nd))]
    else:
        axes = sorted(set(int(a) for a in rng.integers(0, nd, int(rng.integers(1, nd + 1)))))
        if rng.random() < 0.3:
            axes = []
    dev = Dev(lib)
    try:
        nodes, cleaves = [], []
        for L in leaves:
            t = Tensor(L["data"] if L["kind"] != "T" else np.ascontiguousarray(L["data"].T), hip,
                       dtype=DT_NAME[L["dtype"]])
            if L["kind"] == "T":
                t = t.transpose().realize()
            n = t._node
            nodes.append(n)
            if L["kind"] == "scalar":
                cleaves.append((n.data.ptr, L["dtype"], True, [0] * nd))
                continue
            lshape, lst = list(n.view.shape), list(n.view.strides)
            off = nd - len(lshape)
            cleaves.append((n.data.ptr, L["dtype"], False, [0] * off + [0 if e == 1 else s for e, s in zip(lshape, lst)]))
        opc = ob.OpEnum
        for name, a, b, dt in insts:
            if name == "CAST":
                nodes.append(ob.cast(nodes[a], DT_NAME[dt]))
            elif name in BINARY:
                nodes.append(ob._binary(getattr(opc, name), nodes[a], nodes[b]))
            else:
                nodes.append(ob._unary(getattr(opc, name), nodes[a]))
        fn = {SUM: ob.sum, MAX: ob.max, ARGMAX: ob.argmax}[op]
        g = fn(nodes[value], axes if axes else list(range(nd)), False)
        ob.execute_graph(g)
        want = np.asarray(ob.buffer_to_numpy(g.data)).reshape(-1)
        got, _ = run(lib, dev, tuple(shape), cleaves, insts, value, op, tuple(axes))
        got = got.reshape(-1)
        assert got.dtype == want.dtype and np.array_equal(bits(got), bits(want)), (seed, shape, insts, op, axes)
    finally:
        dev.free()
