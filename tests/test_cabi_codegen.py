"""CPU-side checks of the drop-in boundary and the hipRTC code generator.

No GPU is needed: libormi_hip.so loads and reports "no device", hipRTC compiles
generated kernels to gfx950 code objects offline, and the kernel planner runs on
graphs whose leaves live on the CPU oracle device.
"""
import ctypes

import numpy as np
import pytest

from conftest import map_tile_groups, header_functions

ORMI_HIP_OK, ORMI_HIP_ERR_NO_DEVICE, ORMI_HIP_ERR_INVALID, ORMI_HIP_ERR_COMPILE, ORMI_HIP_ERR_UNSUPPORTED = 0, 2, 3, 4, 5


def test_library_exports_every_header_symbol(cabi):
    names = header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(cabi, n)]
    assert not missing, f"declared in include/ormi_hip.h but not exported: {missing}"


def test_no_gpu_reports_no_device(cabi):
    """Without a GPU the device is absent the way a throwing CUDAAllocator makes
    CUDA absent (reference csrc/tests/test_utils.h:17-21)."""
    import os

    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is visible")
    n = ctypes.c_int(-1)
    assert cabi.ormi_hip_device_count(ctypes.byref(n)) == ORMI_HIP_OK and n.value == 0
    assert cabi.ormi_hip_init(0) == ORMI_HIP_ERR_NO_DEVICE
    assert b"no GPU" in cabi.ormi_hip_last_error()


def test_argument_errors_before_device_use(cabi):
    assert cabi.ormi_hip_device_count(None) == ORMI_HIP_ERR_INVALID
    assert cabi.ormi_hip_malloc(None, 16) == ORMI_HIP_ERR_INVALID
    assert cabi.ormi_hip_fill(None, None, 4, 8) == ORMI_HIP_ERR_INVALID
    assert cabi.ormi_hip_convert(None, 0, None, 0, 4) == ORMI_HIP_ERR_INVALID
    assert cabi.ormi_hip_gemm(None) == ORMI_HIP_ERR_INVALID
    assert b"null" in cabi.ormi_hip_last_error()
    # Zero-size work is a no-op that succeeds, as an empty launch is.
    assert cabi.ormi_hip_fill(None, None, 4, 0) == ORMI_HIP_OK
    assert cabi.ormi_hip_memcpy_h2d(None, None, 0) == ORMI_HIP_OK


class GemmDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int),
                ("a", ctypes.c_void_p), ("a_stride_m", ctypes.c_int64), ("a_stride_k", ctypes.c_int64),
                ("b", ctypes.c_void_p), ("b_stride_k", ctypes.c_int64), ("b_stride_n", ctypes.c_int64),
                ("c", ctypes.c_void_p), ("batch_ndim", ctypes.c_int), ("batch_shape", ctypes.c_int * 4),
                ("a_batch_stride", ctypes.c_int64 * 4), ("b_batch_stride", ctypes.c_int64 * 4)]


def test_gemm_descriptor_validation(cabi):
    d = GemmDesc(dtype=0, M=-1, N=4, K=4)
    assert cabi.ormi_hip_gemm(ctypes.byref(d)) == ORMI_HIP_ERR_INVALID
    d = GemmDesc(dtype=5, M=4, N=4, K=4)  # int64 is not a GEMM input type
    assert cabi.ormi_hip_gemm(ctypes.byref(d)) == ORMI_HIP_ERR_UNSUPPORTED
    d = GemmDesc(dtype=0, M=4, N=4, K=4, batch_ndim=5)
    assert cabi.ormi_hip_gemm(ctypes.byref(d)) == ORMI_HIP_ERR_INVALID
    d = GemmDesc(dtype=0, M=0, N=4, K=4)  # empty output: nothing to do
    assert cabi.ormi_hip_gemm(ctypes.byref(d)) == ORMI_HIP_OK
    d = GemmDesc(dtype=0, M=4, N=4, K=4)  # operands are read: null is an error
    assert cabi.ormi_hip_gemm(ctypes.byref(d)) == ORMI_HIP_ERR_INVALID and b"null" in cabi.ormi_hip_last_error()
    d = GemmDesc(dtype=0, M=4, N=4, K=0)  # K == 0 reads no operand, but C is written
    assert cabi.ormi_hip_gemm(ctypes.byref(d)) == ORMI_HIP_ERR_INVALID and b"null" in cabi.ormi_hip_last_error()
    # batch extents whose product overflows 64 bits are refused, not wrapped
    d = GemmDesc(dtype=0, M=4, N=4, K=4, batch_ndim=4)
    for i in range(4):
        d.batch_shape[i] = 1 << 30
    assert cabi.ormi_hip_gemm(ctypes.byref(d)) == ORMI_HIP_ERR_UNSUPPORTED and b"65535" in cabi.ormi_hip_last_error()


class GemmEpilogue(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("fn", ctypes.c_int), ("form", ctypes.c_int), ("s", ctypes.c_void_p),
                ("d", ctypes.c_void_p), ("d_stride_m", ctypes.c_int64), ("d_stride_n", ctypes.c_int64),
                ("d_batch_stride", ctypes.c_int64 * 4), ("aux", ctypes.c_void_p)]


def test_gemm_epilogue_validation(cabi):
    """Malformed epilogues are rejected before any device work (the operand
    pointers are never dereferenced)."""
    base = 1 << 40  # fake, 16-byte aligned device addresses
    d = GemmDesc(dtype=0, M=8, N=8, K=8, a=base, a_stride_m=8, a_stride_k=1, b=base + 4096, b_stride_k=8,
                 b_stride_n=1, c=base + 8192)

    def rc(**kw):
        return cabi.ormi_hip_gemm_ex(ctypes.byref(d), ctypes.byref(GemmEpilogue(**kw)))

    assert rc(kind=9) == ORMI_HIP_ERR_INVALID and b"kind" in cabi.ormi_hip_last_error()
    assert rc(kind=2, fn=42) == ORMI_HIP_ERR_INVALID and b"function" in cabi.ormi_hip_last_error()
    assert rc(kind=1, form=3, d=base + 12288, d_stride_m=8, d_stride_n=1) == ORMI_HIP_ERR_INVALID
    assert rc(kind=1) == ORMI_HIP_ERR_INVALID and b"needs D" in cabi.ormi_hip_last_error()
    assert rc(kind=3, d=base + 12289, d_stride_m=8, d_stride_n=1) == ORMI_HIP_ERR_INVALID
    assert b"aligned" in cabi.ormi_hip_last_error()
    assert rc(kind=2, fn=7, aux=base + 8192 + 64) == ORMI_HIP_ERR_INVALID and b"aux" in cabi.ormi_hip_last_error()
    # D inside C with another layout (transposed) would race; C's own layout is fine.
    assert rc(kind=1, form=1, d=base + 8192, d_stride_m=1, d_stride_n=8) == ORMI_HIP_ERR_INVALID
    assert b"overlaps" in cabi.ormi_hip_last_error()
    empty = GemmDesc(dtype=0, M=0, N=8, K=8)
    assert cabi.ormi_hip_gemm_ex(ctypes.byref(empty), ctypes.byref(GemmEpilogue(kind=2, fn=7))) == ORMI_HIP_OK


def _compile_only(cabi, src: str, opts):
    arr = (ctypes.c_char_p * len(opts))(*[o.encode() for o in opts])
    size = ctypes.c_size_t(0)
    rc = cabi.ormi_hip_rtc_compile_only(src.encode(), b"gfx950", arr, len(opts), ctypes.byref(size))
    return rc, size.value


def test_rtc_compile_only_and_compile_errors(cabi, ob):
    opts = ob._rtc_options()
    rc, size = _compile_only(cabi, 'extern "C" __global__ void k(float* o) { o[threadIdx.x] = 1.0f; }', opts)
    assert rc == ORMI_HIP_OK and size > 0
    rc, _ = _compile_only(cabi, 'extern "C" __global__ void k(float* o) { o[threadIdx.x] = undefined_name; }', opts)
    assert rc == ORMI_HIP_ERR_COMPILE
    assert b"undefined_name" in cabi.ormi_hip_last_error()


def test_fastdiv_matches_integer_division(ob):
    rng = np.random.default_rng(0)
    divisors = [1, 2, 3, 7, 64, 1000, 4096, 8191, 65537, 2 ** 31 - 1, 2 ** 31]
    divisors += [int(v) for v in rng.integers(1, 2 ** 31, 20)]
    for d in divisors:
        m, s = ob._fastdiv(d)
        n = np.concatenate([rng.integers(0, 2 ** 31, 2000, dtype=np.uint64),
                            np.array([0, 1, d - 1, d, d + 1, 2 ** 31 - 1], dtype=np.uint64) % (2 ** 31)])
        q = (((n * np.uint64(m)) >> np.uint64(32)) + n) >> np.uint64(s)
        assert np.array_equal(q, n // np.uint64(d)), d


# ----------------------------------------------------------- code generator
def _cpu(x):
    from ormi_amd import Tensor

    return Tensor(np.asarray(x, np.float32), "cpu")


def test_generated_map_kernel_structure(ob, cpu, cabi):
    """The C2 chain is one kernel with 128-bit operand loads, the broadcast
    operands read per row / per column (no per-element div/mod against literal
    sizes as in reference compiler.cu:76-101), and it compiles for gfx950."""
    X, B, S = _cpu(np.zeros((64, 256))), _cpu(np.zeros(256)), _cpu(np.zeros((64, 1)))
    z = ((X + B) * S).tanh() * X.sigmoid() - 0.1 * X * X
    d = ob._plan_kernel(z._node)
    src = d["source"]
    assert d["plan"].startswith("map") and "vec=4" in d["plan"]
    assert src.count("ormi_f4*") >= 3  # x and bias loads, the output store
    for literal in ("256", "64)"):
        assert f"G = {literal}" not in src
    assert "tanhf" in src or "ormi_tanh" in src
    rc, size = _compile_only(cabi, src, ob._rtc_options())
    assert rc == ORMI_HIP_OK, cabi.ormi_hip_last_error()
    assert size > 0


def row_mode_shapes(tile):
    """(rows, cols) of fp32 maps over a bias row whose tile of `tile` groups of 4
    floats spans whole rows (1), lies inside one row (2: an odd row count), is
    one row (3) or neither (0); with an even row count a tile inside one row
    becomes `unroll` rows of one 256-group window (4)."""
    return {1: [(64, 128), (512, 256)], 3: [(8, 4 * tile), (512, 4 * tile)], 2: [(3, 8 * tile), (5, 12 * tile)],
            4: [(4, 8 * tile), (2, 12 * tile)], 0: [(10, 100), (7, 300)]}


def test_kernel_source_is_shape_independent(ob, cpu):
    """Sizes and strides are arguments: the same chain over another shape of the
    same structure and the same tile alignment to the rows generates the same
    kernel (one cache entry)."""
    def plan(r, c):
        X, B = _cpu(np.zeros((r, c))), _cpu(np.zeros(c))
        return ob._plan_kernel(((X + B) * 2.0).exp()._node)

    names = {}
    for mode, shapes in row_mode_shapes(map_tile_groups(ob)).items():
        a, b = plan(*shapes[0]), plan(*shapes[1])
        assert f"rows={mode}" in a["plan"] and f"rows={mode}" in b["plan"], (a["plan"], b["plan"])
        assert a["name"] == b["name"] and a["source"] == b["source"]
        names[mode] = a["name"]
    assert len(set(names.values())) == 5
    assert plan(64, 128)["name"] != ob._plan_kernel((_cpu(np.zeros((64, 128))) * 2.0).exp()._node)["name"]


def test_row_tiles_keep_a_window_per_block(ob, cpu):
    """Tiles of `unroll` rows: the grid is a multiple of the 256-group windows of
    a row (a block keeps its window while it walks rows), rounded down from the
    64 blocks per CU when there are more tiles; an odd row count keeps one-row
    tiles."""
    tile = map_tile_groups(ob)

    def plan(r, c):
        X, B = _cpu(np.zeros((r, c))), _cpu(np.zeros(c))
        return ob._plan_kernel(((X + B) * 2.0)._node)

    for (r, c), grid in [((6, 12 * tile), 18), ((5472, 12 * tile), 16380), ((8200, 8 * tile), 16384)]:
        d = plan(r, c)
        windows = c // 4 // 256
        assert "rows=4" in d["plan"] and d["grid"][0] == grid and grid % windows == 0, (r, c, d["plan"], d["grid"])
    assert "rows=2" in plan(5471, 12 * tile)["plan"]


@pytest.mark.parametrize("mode", [1, 2, 3, 4, 0])
@pytest.mark.parametrize("variant", ["plain", "3d", "vec1", "multi"])
def test_row_aligned_map_kernels_compile(ob, cpu, cabi, mode, variant):
    """Every tile alignment compiles for gfx950: two dims and three (outer
    coordinates by division), 1-float groups (a transposed operand, with the
    row length in floats set so the alignment holds) and several outputs from
    one kernel."""
    tile = map_tile_groups(ob)
    r, c = row_mode_shapes(tile)[mode][0]
    if variant == "vec1" and mode in (2, 3, 4):
        c //= 4
    x, bias, scale = _cpu(np.ones((r, c))), _cpu(np.ones(c)), _cpu(np.ones((r, 1)))
    if variant == "3d":  # 3 r rows: odd for mode 2, even for mode 4
        x = _cpu(np.ones((3, 1, c))) * _cpu(np.ones((1, r, c)))
        scale = _cpu(np.ones((3, r, 1)))
    z = ((x + bias) * scale - x * 0.5)._node
    if variant == "vec1":
        z = ob.add(z, _view_leaf(ob, np.ones(r * c), [r, c], [1, r]))
    if variant == "multi":
        d = ob._plan_group([z, (x * scale)._node])
    else:
        d = ob._plan_kernel(z)
    if variant == "3d":
        assert "ndim=3" in d["plan"], d["plan"]
    assert f"rows={mode}" in d["plan"] and ("vec=1" in d["plan"]) == (variant == "vec1"), d["plan"]
    rc, _ = _compile_only(cabi, d["source"], ob._rtc_options())
    assert rc == ORMI_HIP_OK, (d["plan"], cabi.ormi_hip_last_error())


@pytest.mark.parametrize("axes,kind", [((1,), "row"), ((0,), "col")])
def test_generated_reduction_kernels_compile(ob, cpu, cabi, axes, kind):
    x = _cpu(np.zeros((1024, 2048)))
    for red in ("sum", "max", "argmax"):
        node = getattr(ob, red)((x * 2.0)._node, list(axes), False)
        d = ob._plan_kernel(node)
        assert kind in d["plan"], d["plan"]
        rc, _ = _compile_only(cabi, d["source"], ob._rtc_options())
        assert rc == ORMI_HIP_OK, (red, cabi.ormi_hip_last_error())
        if d["two_pass"]:
            rc, _ = _compile_only(cabi, d["second_source"], ob._rtc_options())
            assert rc == ORMI_HIP_OK, (red, cabi.ormi_hip_last_error())


def test_long_axis_reduction_is_two_pass(ob, cpu):
    """A global reduction (few outputs, long axis) is split across work-groups
    and finished by a second kernel in part order: deterministic, no atomics
    (the reference's atomicAdd per element, cuda/kernels/reduce/sum.cu:65)."""
    x = _cpu(np.zeros((4096, 4096)))
    d = ob._plan_kernel(ob.sum(x._node, [0, 1], False))
    assert d["two_pass"] and d["workspace_bytes"] > 0
    assert "atomic" not in d["source"] and "atomic" not in d["second_source"]


def test_multi_output_group_plan(ob, cpu, cabi):
    """Sibling element-wise roots of one shape plan as ONE kernel with one output
    each; shared interior nodes are computed once (fewer instructions than the
    separate tapes), and the kernel compiles for gfx950."""
    rng = np.random.default_rng(5)
    a, b, c = (_cpu(rng.standard_normal((64, 256))) for _ in range(3))
    h = a * b + c
    roots = [h.relu() * b, h.relu() * a, h.relu(), a - c]
    d = ob._plan_group([r._node for r in roots])
    assert "outputs=4" in d["plan"], d["plan"]
    assert d["num_leaves"] == 3
    separate = sum(ob._plan_group([r._node])["num_insts"] for r in roots)
    assert d["num_insts"] < separate
    for r in range(4):
        assert f"out{r}" in d["source"]
    rc, _ = _compile_only(cabi, d["source"], ob._rtc_options())
    assert rc == ORMI_HIP_OK, cabi.ormi_hip_last_error()
    # A single root keeps the single-output kernel (same source as _plan_kernel).
    assert ob._plan_group([roots[0]._node])["source"] == ob._plan_kernel(roots[0]._node)["source"]


def test_realize_all_on_cpu_realizes_each(cpu):
    """Devices without a group scheduler (the CPU oracle) realize each node."""
    from ormi_amd import Tensor, realize_all

    x = Tensor(np.arange(6, dtype=np.float32).reshape(2, 3), "cpu")
    y, z = x * 2.0, (x + 1.0).sum(1)
    realize_all(y, z, y)
    assert y._node.is_realized and z._node.is_realized
    assert y.numpy().tolist() == [[0, 2, 4], [6, 8, 10]] and z.numpy().tolist() == [6, 15]


def test_allocator_size_classes(ob):
    """Powers of two from 512 B to 1 MiB, then multiples of 2 MiB."""
    MiB = 1 << 20
    cases = {0: 512, 1: 512, 512: 512, 513: 1024, 4000: 4096, 4096: 4096, 4097: 8192, MiB: MiB,
             MiB + 1: 2 * MiB, 3 * MiB: 4 * MiB, 128 * MiB: 128 * MiB, 128 * MiB + 16384: 130 * MiB}
    for n, c in cases.items():
        assert ob._size_class(n) == c, (n, ob._size_class(n), c)
    rng = np.random.default_rng(3)
    for n in rng.integers(1, 1 << 31, 200):
        c = ob._size_class(int(n))
        assert c >= n and (c < 2 * n or c == 512 or c - n < 2 * MiB)


def _view_leaf(ob, arr, shape, strides):
    buf = ob.numpy_to_buffer(np.ascontiguousarray(arr, np.float32).reshape(-1), ob.DeviceEnum.CPU)
    n = ob.Node(buf, False, ob.Device(ob.DeviceEnum.CPU, 0))
    n.view = ob.TensorView(list(shape), list(strides))
    return n


@pytest.mark.parametrize("kind", ["bcast3", "bcast4", "transposed3", "reduce3"])
def test_generated_kernels_compile_for_nd_index_spaces(ob, cpu, cabi, kind):
    """Index spaces that keep 3-4 dims after merging (non-mergeable broadcasts,
    transposed views): every generated kernel compiles for gfx950. A repeated
    quotient declaration in the index decomposition once broke exactly these."""
    if kind == "bcast3":
        node = ob.mul(_cpu(np.ones((4, 33, 1)))._node, _cpu(np.ones((1, 33, 3)))._node)
    elif kind == "bcast4":
        node = ob.add(_cpu(np.ones((2, 1, 5, 1)))._node, _cpu(np.ones((1, 3, 1, 7)))._node)
    elif kind == "transposed3":
        x = _view_leaf(ob, np.ones(16 * 33 * 64), [64, 33, 16], [1, 64, 33 * 64])
        node = ob.sin(x)
    else:
        x = _view_leaf(ob, np.ones(16 * 33 * 64), [64, 33, 16], [1, 64, 33 * 64])
        node = ob.sum(ob.exp(x), [1], False)
    d = ob._plan_kernel(node)
    rc, _ = _compile_only(cabi, d["source"], ob._rtc_options())
    assert rc == ORMI_HIP_OK, (d["plan"], cabi.ormi_hip_last_error())
    if d["two_pass"]:
        rc, _ = _compile_only(cabi, d["second_source"], ob._rtc_options())
        assert rc == ORMI_HIP_OK, cabi.ormi_hip_last_error()


def test_map_and_reduce_plans_past_2_31_use_64_bit_indices(ob, cpu):
    """A broadcast map over 65537 x 32768 elements (> 2^31; the operands are a
    row and a column, so nothing large is allocated) plans 64-bit indices and
    no 32-bit byte offsets; a small one plans 32-bit offsets."""
    from ormi_amd import Tensor

    a = Tensor(np.zeros(32768, np.float32), "cpu")
    b = Tensor(np.zeros((65537, 1), np.float32), "cpu")
    plan = ob._plan_kernel((b + a)._node)["plan"]
    assert "idx=64" in plan and "off32=0" in plan
    small = ob._plan_kernel((Tensor(np.zeros((4, 1), np.float32), "cpu") + a)._node)["plan"]
    assert "idx=32" in small and "off32=1" in small


def test_column_kernels_keyed_by_column_waves(ob, cpu, cabi):
    """A column reduction's waves across columns follow the kept extent (1 for 6
    columns, 2 for 70, 8 for 2048), and the emitted body depends on it, so the
    kernel cache keys it: a narrow plan compiled first must not serve a wider one
    whose grid assumes more columns per block."""
    seen = {}
    for shape in [(1 << 16, 6), (1003, 70), (1024, 2048)]:
        for red in ("sum", "argmax"):
            d = ob._plan_kernel(getattr(ob, red)(_cpu(np.zeros(shape))._node, [0], False))
            cw = int(d["plan"].split("cwaves=")[1].split()[0])
            assert f"bi_ * {64 * cw} + cl" in d["source"], (shape, red, d["plan"])
            seen.setdefault(red, set()).add(d["name"])
            rc, _ = _compile_only(cabi, d["source"], ob._rtc_options())
            assert rc == ORMI_HIP_OK, (shape, red, cabi.ormi_hip_last_error())
    assert all(len(names) == 3 for names in seen.values()), seen


def test_long_rows_share_waves(ob, cpu, cabi):
    """Rows of at least 1024 groups, enough of them for one pass, are shared by
    four waves of a block that combine through LDS in wave order; shorter rows
    and split rows keep one wave per (row, part). The two layouts are different
    kernels (the name carries the wave count) and both compile."""
    def plan(shape, red):
        return ob._plan_kernel(getattr(ob, red)(_cpu(np.zeros(shape))._node, [1], False))

    for red in ("sum", "max", "argmax"):
        long_rows, short_rows, split = plan((4099, 4108), red), plan((4099, 4092), red), plan((64, 8192), red)
        assert "waves_per_row=4" in long_rows["plan"] and "__syncthreads()" in long_rows["source"], long_rows["plan"]
        assert "waves_per_row=1" in short_rows["plan"] and "__syncthreads()" not in short_rows["source"]
        assert "waves_per_row=1" in split["plan"] and split["two_pass"], split["plan"]
        assert long_rows["name"] != short_rows["name"]
        for d in (long_rows, short_rows):
            rc, _ = _compile_only(cabi, d["source"], ob._rtc_options())
            assert rc == ORMI_HIP_OK, (red, d["plan"], cabi.ormi_hip_last_error())


def test_non_temporal_loads_only_for_large_read_once_operands(ob, cpu):
    """Loads carry the non-temporal hint only for operands read once (no zero
    stride), and only when those bring in at least 64 MiB: the C2 chain's
    (8192, 4096) input is hinted, its bias row (re-read by every row) is not,
    and a (1024, 4096) chain or row sum is not hinted at all."""
    def body(d):
        return d["source"].split('extern "C"')[1]

    x, bias = np.zeros((8192, 4096), np.float32), np.zeros(4096, np.float32)
    d = ob._plan_kernel((_cpu(x) + _cpu(bias)).tanh()._node)
    src = body(d)
    assert src.count("__builtin_nontemporal_load(") == 1, src
    assert "__builtin_nontemporal_load((const ormi_f4*)((const char*)L0" in src, src
    small = body(ob._plan_kernel((_cpu(x[:1024]) + _cpu(bias)).tanh()._node))
    assert "__builtin_nontemporal_load(" not in small
    assert "__builtin_nontemporal_load(" in body(ob._plan_kernel(ob.sum(_cpu(x)._node, [1], False)))
    assert "__builtin_nontemporal_load(" not in body(ob._plan_kernel(ob.sum(_cpu(x[:1024])._node, [1], False)))


def test_large_streams_cap_work_groups_per_cu(ob, cpu):
    """Map and row-reduction kernels whose grid would put more work-groups on
    a CU than the measured best (5 for maps, 3 for row sums, 4 for row max /
    argmax) get dynamic LDS that leaves room for only that many of them
    (160 KB per CU, 1 KB kept for the kernel's own LDS). Small grids, maps
    that mostly read, and rows that one wave covers get none."""
    def lds(d):
        return d["lds"]

    def cap(n):
        return (160 * 1024 // n - 1024) // 512 * 512

    x = np.zeros((8192, 4096), np.float32)
    big_map = ob._plan_kernel((_cpu(x) * 2.0)._node)
    assert lds(big_map) == cap(5) and f"lds={cap(5)}" in big_map["plan"]
    assert 5 * (cap(5) + 512) <= 160 * 1024 < 6 * cap(5)
    assert lds(ob._plan_kernel((_cpu(x[:512]) * 2.0)._node)) == 0   # 512 work-groups: 2 per CU
    assert lds(ob._plan_kernel(ob.sum(_cpu(x)._node, [1], False))) == cap(3)
    assert lds(ob._plan_kernel(ob.max(_cpu(x)._node, [1], False))) == cap(4)
    assert lds(ob._plan_kernel(ob.sum(_cpu(x[:256])._node, [1], False))) == 0
    y, z = np.ones((8192, 4096), np.float32), np.full((8192, 4096), 2.0, np.float32)
    assert lds(ob._plan_kernel((_cpu(x) + _cpu(y) + _cpu(z))._node)) == 0  # reads 3x what it writes
    short = ob._plan_kernel(ob.sum(_cpu(np.zeros((65536, 512), np.float32))._node, [1], False))
    assert "waves_per_row=1" in short["plan"] and lds(short) == 0


def test_kernel_cache_tells_bf16_from_f16(ob, cpu):
    """bf16 and fp16 share a storage type (unsigned short). The generator's
    kernel cache must still key on the element type: a bf16 leaf (or output)
    planned after an otherwise identical fp16 one gets its own kernel, with its
    own conversion. Before the element types were in the key, the second plan
    reused the first kernel and read bf16 bits as fp16."""
    from ormi_amd import Tensor

    a = np.linspace(-2, 2, 8 * 64, dtype=np.float32).reshape(8, 64)
    p16 = ob._plan_kernel(Tensor(a, "cpu", dtype="float16").tanh()._node)
    pbf = ob._plan_kernel(Tensor(a, "cpu", dtype="bfloat16").tanh()._node)
    assert p16["name"] != pbf["name"]
    assert "ormi_f16_to_f32(" in p16["source"] and "ormi_bf16_to_f32(" not in p16["source"].split("extern")[1]
    assert "ormi_bf16_to_f32(" in pbf["source"].split("extern")[1]
    o16 = ob._plan_kernel((Tensor(a, "cpu") * 2.0).astype("float16")._node)
    obf = ob._plan_kernel((Tensor(a, "cpu") * 2.0).astype("bfloat16")._node)
    assert o16["name"] != obf["name"]
    assert "ormi_f32_to_bf16(" in obf["source"].split("extern")[1]
    assert "ormi_f32_to_bf16(" not in o16["source"].split("extern")[1]


def test_planner_walks_large_regions(ob, cpu):
    """A region wider and deeper than the planner's inline walk storage (32
    visited nodes, 64 stack entries before they move to the heap): a chain
    v[k+1] = v[k] * v[k-1] + leaf[k] over 150 distinct leaves, so every value
    is shared by two consumers. The tape holds each leaf and each node once,
    and a second root inside the first one's region adds nothing."""
    n = 150
    leaves = [_cpu(np.full((4, 8), 1.0 + k / n)) for k in range(n + 2)]
    v = [leaves[0], leaves[1]]
    for k in range(n):
        v.append(v[-1] * v[-2] + leaves[k + 2])
    root = v[-1]._node
    d = ob._plan_group([root])
    assert d["num_leaves"] == n + 2
    assert d["num_insts"] == 2 * n
    both = ob._plan_group([root, v[n // 2]._node])
    assert both["num_leaves"] == n + 2 and both["num_insts"] == 2 * n
    single = ob._plan_kernel(root)
    assert single["num_args"] > n + 2  # every leaf's pointer is an argument
