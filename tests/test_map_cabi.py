"""ormi_hip_map, the C-ABI element-wise entry: a caller's tape (leaves with
strides aligned to the map's shape, instructions over earlier values) becomes
one generated kernel. It replaces the reference's cuda::execute_jit over the
tape of csrc/backend/cuda/compiler.cu:22-51 (jit.cu:13-44).

The same code generator and lowerings serve the graph path, so the C-ABI must
give the graph path's results bit for bit on every tape (random tapes over
every op, broadcast / transposed / scalar / 16-bit leaves, several outputs of
mixed dtypes), and the graph path is itself checked against the CPU oracle in
test_hip_parity.py. Argument checking runs before any device call, so those
tests run without a GPU."""
import ctypes

import numpy as np
import pytest

MAXD = 8
F32, I32, BOOL, BF16, F16, I64 = 0, 1, 2, 3, 4, 5
NAMES = ["NEG", "EXP", "LOG", "SIN", "COS", "ADD", "SUB", "MUL", "DIV", "POW", "RELU", "STEP", "TANH", "TANH_GRAD",
         "SIGMOID", "SIGMOID_GRAD", "GELU", "GELU_GRAD", "EQ", "CAST"]
CODE = {n: i for i, n in enumerate(NAMES)}
BINARY = {"ADD", "SUB", "MUL", "DIV", "POW", "EQ"}
UNARY = [n for n in NAMES if n not in BINARY and n != "CAST"]
DT_NAME = {F32: "float32", BF16: "bfloat16", F16: "float16", I64: "int64", I32: "int32", BOOL: "bool"}


class Leaf(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("dtype", ctypes.c_int), ("scalar", ctypes.c_int),
                ("strides", ctypes.c_int64 * MAXD)]


class Inst(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int), ("a", ctypes.c_int), ("b", ctypes.c_int), ("dtype", ctypes.c_int)]


class Desc(ctypes.Structure):
    _fields_ = [("ndim", ctypes.c_int), ("shape", ctypes.c_int * MAXD), ("num_leaves", ctypes.c_int),
                ("leaves", ctypes.POINTER(Leaf)), ("num_insts", ctypes.c_int), ("insts", ctypes.POINTER(Inst)),
                ("num_outputs", ctypes.c_int), ("output_values", ctypes.POINTER(ctypes.c_int)),
                ("outputs", ctypes.POINTER(ctypes.c_void_p)), ("output_dtypes", ctypes.POINTER(ctypes.c_int))]


def make_desc(shape, leaves, insts, outputs):
    """leaves: (ptr, dtype, scalar, strides); insts: (op name, a, b, dtype);
    outputs: (value, ptr, dtype). Returns the descriptor and what keeps its
    arrays alive."""
    L = (Leaf * max(1, len(leaves)))()
    for i, (ptr, dt, sc, st) in enumerate(leaves):
        L[i].ptr, L[i].dtype, L[i].scalar = ptr, dt, int(sc)
        for k, s in enumerate(st):
            L[i].strides[k] = s
    I = (Inst * max(1, len(insts)))()
    for i, (op, a, b, dt) in enumerate(insts):
        I[i].op, I[i].a, I[i].b, I[i].dtype = CODE[op] if isinstance(op, str) else op, a, b, dt
    vals = (ctypes.c_int * len(outputs))(*[o[0] for o in outputs])
    outs = (ctypes.c_void_p * len(outputs))(*[o[1] for o in outputs])
    dts = (ctypes.c_int * len(outputs))(*[o[2] for o in outputs])
    d = Desc(ndim=len(shape), num_leaves=len(leaves), leaves=L, num_insts=len(insts), insts=I,
             num_outputs=len(outputs), output_values=vals, outputs=outs, output_dtypes=dts)
    for k, e in enumerate(shape):
        d.shape[k] = e
    return d, (L, I, vals, outs, dts)


@pytest.fixture(scope="module")
def mapc(cabi):
    cabi.ormi_hip_map.argtypes = [ctypes.POINTER(Desc)]
    return cabi


# ----------------------------------------------------------------- no GPU --
@pytest.mark.parametrize("case,msg", [
    (dict(ndim=9), b"ndim must be 0..8"),
    (dict(shape=(4, -1)), b"negative extent"),
    (dict(shape=(1 << 30,) * 3), b"more than 2^62 elements"),
    (dict(leaf_dtype=9), b"leaf 0 has an unknown dtype"),
    (dict(op=77), b"instruction 0 has an unknown op"),
    (dict(a=1), b"operand a must be an earlier value"),
    (dict(op="ADD", b=5), b"operand b must be an earlier value"),
    (dict(op="CAST", cast=I64), b"CAST rounds to bf16, f16 or f32 only"),
    (dict(out_value=7), b"output 0 names no value"),
    (dict(out_dtype=-1), b"output 0 has an unknown dtype"),
    (dict(num_outputs=0), b"num_outputs must be 1..16"),
    (dict(null_leaf=True), b"leaf 0 is null"),
    (dict(null_out=True), b"output 0 is null"),
    (dict(leaf_ptr=0x1002), b"leaf 0 is not aligned to its element size"),
    (dict(out_ptr=0x2001), b"output 0 is not aligned to its element size"),
])
def test_map_rejects_bad_descriptors(mapc, case, msg):
    shape = case.get("shape", (4, 8))
    leaves = [(None if case.get("null_leaf") else case.get("leaf_ptr", 0x1000), case.get("leaf_dtype", F32), False, (8, 1))]
    insts = [(case.get("op", "NEG"), case.get("a", 0), case.get("b", 0), case.get("cast", F32))]
    outs = [(case.get("out_value", 1), None if case.get("null_out") else case.get("out_ptr", 0x2000), case.get("out_dtype", F32))]
    d, keep = make_desc(shape, leaves, insts, outs)
    if "ndim" in case:
        d.ndim = case["ndim"]
    if "num_outputs" in case:
        d.num_outputs = case["num_outputs"]
    assert mapc.ormi_hip_map(ctypes.byref(d)) == 3  # ORMI_HIP_ERR_INVALID
    assert msg in mapc.ormi_hip_last_error()


def test_map_of_an_empty_shape_is_a_no_op(mapc):
    d, keep = make_desc((0, 8), [(0x1000, F32, False, (8, 1))], [("EXP", 0, 0, F32)], [(1, 0x2000, F32)])
    assert mapc.ormi_hip_map(ctypes.byref(d)) == 0


# -------------------------------------------------------------------- GPU --
class Dev:
    def __init__(self, lib):
        self.lib, self.ptrs = lib, []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.lib.ormi_hip_malloc(ctypes.byref(p), max(nbytes, 4)) == 0
        self.ptrs.append(p)
        return p.value

    def get(self, p, nbytes):
        out = np.empty(nbytes, np.uint8)
        assert self.lib.ormi_hip_memcpy_d2h(out.ctypes.data, ctypes.c_void_p(p), nbytes) == 0
        return out

    def free(self):
        for p in self.ptrs:
            self.lib.ormi_hip_free(p)


def widen(raw: np.ndarray, dt: int, n: int) -> np.ndarray:
    """Bytes of n stored values of dtype dt -> float64 (integers) or float32 bits."""
    if dt == F32:
        return raw.view(np.float32)[:n]
    if dt == BF16:
        return (raw.view(np.uint16)[:n].astype(np.uint32) << 16).view(np.float32)
    if dt == F16:
        return raw.view(np.float16)[:n].astype(np.float32)
    return raw.view({I64: np.int64, I32: np.int32, BOOL: np.uint8}[dt])[:n]


def graph_result(ob, node, dt, shape):
    """The realized node's values at the map's shape: a value that depends only
    on broadcast leaves has a smaller shape in the graph (numpy's broadcasting),
    while the map writes it at every position."""
    a = np.asarray(ob.buffer_to_numpy(node.data)).reshape(tuple(node.view.shape))
    a = np.broadcast_to(a, tuple(shape)).reshape(-1)
    return a.astype(np.uint8) if dt == BOOL else a


def same_bits(a, b):
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.astype(np.float32).view(np.uint32))
    return np.array_equal(a, b.astype(a.dtype))


def random_case(seed):
    rng = np.random.default_rng(seed)
    ndim = int(rng.integers(1, 4))
    shape = [int(rng.choice([1, 3, 8, 17, 64, 129, 512])) for _ in range(ndim)]
    while int(np.prod(shape)) > 400_000:
        shape[int(np.argmax(shape))] //= 4
    leaves = []
    for _ in range(int(rng.integers(2, 6))):
        kind = rng.random()
        dt = int(rng.choice([F32, F32, BF16, F16]))
        if kind < 0.15:
            leaves.append(dict(kind="scalar", dtype=dt, data=np.float32(rng.uniform(-2, 2))))
            continue
        # right-aligned: drop some leading dims, make some dims 1 (broadcast)
        drop = int(rng.integers(0, ndim)) if rng.random() < 0.3 else 0
        lshape = [1 if rng.random() < 0.3 else e for e in shape[drop:]]
        transposed = len(lshape) == 2 and rng.random() < 0.3
        leaves.append(dict(kind="T" if transposed else "plain", dtype=dt,
                           data=rng.uniform(-2, 2, lshape).astype(np.float32)))
    nl = len(leaves)
    insts = []
    for k in range(int(rng.integers(3, 11))):
        nv = nl + k
        r = rng.random()
        a = int(rng.integers(0, nv)) if rng.random() < 0.5 else nv - 1
        if r < 0.45:
            insts.append((str(rng.choice(UNARY)), a, -1, F32))
        elif r < 0.9:
            insts.append((str(rng.choice(sorted(BINARY))), a, int(rng.integers(0, nv)), F32))
        else:
            insts.append(("CAST", a, -1, int(rng.choice([BF16, F16]))))
    nv = nl + len(insts)
    nout = int(rng.integers(1, 4))
    vals = sorted(set([nv - 1] + [int(v) for v in rng.integers(nl, nv, nout - 1)]))
    outs = [(v, int(rng.choice([F32, F32, BF16, F16, I64, I32, BOOL]))) for v in vals]
    return shape, leaves, insts, outs


def run_both(ob, mapc, dev, shape, leaves, insts, outs):
    """The tape through the graph path (realize_all) and through ormi_hip_map on
    the same leaf buffers; returns [(graph values, C-ABI values)] per output."""
    from ormi_amd import Tensor

    op = ob.OpEnum
    nodes, cleaves = [], []
    for L in leaves:
        t = Tensor(L["data"] if L["kind"] != "T" else np.ascontiguousarray(L["data"].T), "hip",
                   dtype=DT_NAME[L["dtype"]])
        if L["kind"] == "T":
            t = t.transpose().realize()  # a view: realizing aliases the buffer
        n = t._node
        nodes.append(n)
        if L["kind"] == "scalar":
            cleaves.append((n.data.ptr, L["dtype"], True, [0] * len(shape)))
            continue
        lshape, lst = list(n.view.shape), list(n.view.strides)
        off = len(shape) - len(lshape)
        st = [0] * off + [0 if e == 1 else s for e, s in zip(lshape, lst)]
        cleaves.append((n.data.ptr, L["dtype"], False, st))
    for name, a, b, dt in insts:
        if name == "CAST":
            nodes.append(ob.cast(nodes[a], DT_NAME[dt]))
        elif name in BINARY:
            nodes.append(ob._binary(getattr(op, name), nodes[a], nodes[b]))
        else:
            nodes.append(ob._unary(getattr(op, name), nodes[a]))
    roots = [nodes[v] if dt == F32 else ob.cast(nodes[v], DT_NAME[dt]) for v, dt in outs]
    ob.realize_all(roots)
    n = int(np.prod(shape))
    size = {F32: 4, BF16: 2, F16: 2, I64: 8, I32: 4, BOOL: 1}
    bufs = [dev.alloc(n * size[dt]) for _, dt in outs]
    d, keep = make_desc(shape, cleaves, insts, [(v, p, dt) for (v, dt), p in zip(outs, bufs)])
    assert mapc.ormi_hip_map(ctypes.byref(d)) == 0, mapc.ormi_hip_last_error()
    res = []
    for (v, dt), r, p in zip(outs, roots, bufs):
        g = graph_result(ob, r, dt, shape)
        res.append((g, widen(dev.get(p, n * size[dt]), dt, n)))
    return res


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(40))
def test_random_tapes_match_the_graph_path_bit_for_bit(ob, mapc, hip, seed):
    shape, leaves, insts, outs = random_case(seed)
    dev = Dev(mapc)
    try:
        for k, (g, c) in enumerate(run_both(ob, mapc, dev, shape, leaves, insts, outs)):
            assert same_bits(c, g), (seed, shape, insts, outs, k)
    finally:
        dev.free()


@pytest.mark.gpu
def test_c2_chain_is_the_graph_kernel(ob, mapc, hip):
    """The C2 chain at full size, tape in the graph path's own order: the
    C-ABI call compiles nothing new (the same kernel text is in the cache) and
    gives the same bits."""
    from ormi_amd import Tensor

    op = ob.OpEnum
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (8192, 4096)).astype(np.float32)
    bias = rng.normal(0, 0.1, (4096,)).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, (8192, 1)).astype(np.float32)
    X, Bi, S = Tensor(x, hip)._node, Tensor(bias, hip)._node, Tensor(scale, hip)._node
    c = Tensor(np.array(0.1, np.float32), hip)._node
    # post-order of build_expr: leaves as first met, instructions after their operands
    t0 = ob._binary(op.ADD, X, Bi)
    t1 = ob._binary(op.MUL, t0, S)
    t2 = ob._unary(op.TANH, t1)
    t3 = ob._unary(op.SIGMOID, X)
    t4 = ob._binary(op.MUL, t2, t3)
    t5 = ob._binary(op.MUL, c, X)
    t6 = ob._binary(op.MUL, t5, X)
    z = ob._binary(op.SUB, t4, t6)
    ob.realize_all([z])
    want = np.asarray(ob.buffer_to_numpy(z.data))
    count = ctypes.c_uint64()
    mapc.ormi_hip_rtc_cache_size.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    assert mapc.ormi_hip_rtc_cache_size(ctypes.byref(count)) == 0
    before = count.value
    dev = Dev(mapc)
    try:
        out = dev.alloc(x.nbytes)
        leaves = [(X.data.ptr, F32, False, [4096, 1]), (Bi.data.ptr, F32, False, [0, 1]),
                  (S.data.ptr, F32, False, [1, 0]), (c.data.ptr, F32, True, [0, 0])]
        insts = [("ADD", 0, 1, F32), ("MUL", 4, 2, F32), ("TANH", 5, -1, F32), ("SIGMOID", 0, -1, F32),
                 ("MUL", 6, 7, F32), ("MUL", 3, 0, F32), ("MUL", 9, 0, F32), ("SUB", 8, 10, F32)]
        d, keep = make_desc((8192, 4096), leaves, insts, [(11, out, F32)])
        assert mapc.ormi_hip_map(ctypes.byref(d)) == 0, mapc.ormi_hip_last_error()
        got = widen(dev.get(out, x.nbytes), F32, x.size).reshape(x.shape)
        assert mapc.ormi_hip_rtc_cache_size(ctypes.byref(count)) == 0
        assert count.value == before, "the C-ABI tape compiled a kernel the graph path did not"
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        dev.free()


@pytest.mark.gpu
def test_negative_strides_and_zero_dims(ob, mapc, hip):
    """A row read backwards (negative stride), a 0-d map, and a leaf that is an
    output of the identity tape (a copy with a dtype change)."""
    rng = np.random.default_rng(5)
    a = rng.standard_normal((64, 300)).astype(np.float32)
    dev = Dev(mapc)
    try:
        pa = dev.alloc(a.nbytes)
        assert mapc.ormi_hip_memcpy_h2d(ctypes.c_void_p(pa), a.ctypes.data, a.nbytes) == 0
        out = dev.alloc(a.nbytes)
        # rev[i, j] = a[i, 299 - j]: base at the last column, stride -1 along j
        leaves = [(pa + 299 * 4, F32, False, [300, -1])]
        d, keep = make_desc((64, 300), leaves, [("NEG", 0, -1, F32)], [(1, out, F32)])
        assert mapc.ormi_hip_map(ctypes.byref(d)) == 0, mapc.ormi_hip_last_error()
        got = widen(dev.get(out, a.nbytes), F32, a.size).reshape(a.shape)
        assert np.array_equal(got, -a[:, ::-1])
        # 0-d: one element
        o1 = dev.alloc(4)
        d, keep = make_desc((), [(pa, F32, True, [])], [("EXP", 0, -1, F32)], [(1, o1, F32)])
        assert mapc.ormi_hip_map(ctypes.byref(d)) == 0, mapc.ormi_hip_last_error()
        g1 = widen(dev.get(o1, 4), F32, 1)[0]
        assert abs(float(g1) - float(np.exp(np.float64(a[0, 0])))) <= 4e-7 * float(np.exp(np.float64(a[0, 0])))
        # identity tape: leaf 0 stored as int64 (ormi_f32_to_i64 on the store)
        o2 = dev.alloc(a.size * 8)
        d, keep = make_desc((64, 300), [(pa, F32, False, [300, 1])], [], [(0, o2, I64)])
        assert mapc.ormi_hip_map(ctypes.byref(d)) == 0, mapc.ormi_hip_last_error()
        g2 = widen(dev.get(o2, a.size * 8), I64, a.size).reshape(a.shape)
        assert np.array_equal(g2, np.trunc(a).astype(np.int64))
    finally:
        dev.free()
