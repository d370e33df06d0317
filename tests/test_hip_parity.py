"""HIP device parity against the CPU oracle (and float64 closed forms at full size).

Tolerances (from the north star): bit-exact for argmax and max, rtol 1e-6 for
fp32 pointwise (atol 1e-6 floor for values near 0, where a 1-ulp transcendental
difference dominates), rtol 1e-5 for fp32 reductions (atol from the summation
error bound), rtol 2e-2 for bf16 GEMM (reference computed from the bf16-rounded
inputs; atol 1e-3 of the output scale).
"""
import math

import numpy as np
import pytest

from conftest import empty_tensor_cases, fp32_sum_tolerance, map_tile_groups

pytestmark = pytest.mark.gpu


def T(data, dev, **kw):
    from ormi_amd import Tensor

    return Tensor(data, device=dev, **kw)


def both(x, **kw):
    return T(x, "cpu", **kw), T(x, "hip", **kw)


def assert_bits_equal(a, b):
    assert a.dtype == b.dtype and a.shape == b.shape
    assert np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


# ----------------------------------------------------------------- KATs on HIP
def test_reference_kats_on_hip(cpu, hip):
    a, b = T([4.0, 6.0], hip), T([2.0, 3.0], hip)
    assert (a + b).numpy().tolist() == [6, 9]
    assert (a - b).numpy().tolist() == [2, 3]
    assert (a * b).numpy().tolist() == [8, 18]
    assert (a / b).numpy().tolist() == [2, 2]
    assert (-a).numpy().tolist() == [-4, -6]
    assert (a ** 2.0).numpy().tolist() == [16, 36]
    a = T([2.0, 4.0], hip)
    assert (10.0 - a).numpy().tolist() == [8, 6]
    assert (10.0 / a).numpy().tolist() == [5, 2.5]
    m = T([[1.0, 2.0], [3.0, 4.0]], hip) @ T([[2.0, 0.0], [0.0, 2.0]], hip)
    assert m.numpy().tolist() == [[2, 4], [6, 8]]
    x = T([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], hip)
    assert x.reshape((3, 2)).numpy().tolist() == [[1, 2], [3, 4], [5, 6]]
    assert x.transpose().numpy().tolist() == [[1, 4], [2, 5], [3, 6]]
    assert x.sum().numpy() == 21.0 and x.sum(1).numpy().tolist() == [6, 15]
    assert x.sum(0, keepdims=True).numpy().tolist() == [[5, 7, 9]]
    cube = T(np.arange(1, 9, dtype=np.float32).reshape(2, 2, 2), hip)
    assert cube.sum((0, 2)).numpy().tolist() == [14, 22]
    a, b = T([2.0, 3.0], hip, requires_grad=True), T([4.0, 5.0], hip, requires_grad=True)
    ((a * b) + a).backward()
    assert a.grad.numpy().tolist() == [5, 6] and b.grad.numpy().tolist() == [2, 3]
    s = T(np.full(2, 1.570796327, np.float32), hip).sin().numpy()
    assert np.allclose(s, 1.0, atol=1e-5)


def test_golden_kats_on_hip(ob, hip):
    """Every vector of tests/golden/reference_kats.json on the HIP device."""
    from kat_runner import cases, run_case

    for case in cases():
        run_case(ob, case, ob.DeviceEnum.HIP)


def test_matmul_kats_on_hip(ob, hip):
    def view(vals, shape, strides):
        buf = ob.numpy_to_buffer(np.array(vals, np.float32), ob.DeviceEnum.HIP)
        n = ob.Node(buf, False, ob.Device(ob.DeviceEnum.HIP, 0))
        n.view = ob.TensorView(list(shape), list(strides))
        return n

    def run(a, b):
        c = ob.matmul(a, b)
        ob.execute_graph(c)
        return ob.buffer_to_numpy(c.data).reshape(-1).tolist()

    assert run(view([1, 2, 3, 4, 5, 6], [2, 3], [3, 1]), view([7, 8, 9, 10, 11, 12], [3, 2], [2, 1])) == [58, 64, 139, 154]
    assert run(view([1, 2, 3, 4, 5, 6], [3, 2], [1, 3]), view([1, 2, 3, 4], [2, 2], [2, 1])) == [13, 18, 17, 24, 21, 30]
    assert run(view(list(range(1, 13)), [2, 2, 3], [6, 3, 1]), view([1, 2, 3, 4, 5, 6], [2, 3, 2], [0, 2, 1])) == \
        [22, 28, 49, 64, 76, 100, 103, 136]


def test_fusion_contract(ob, hip):
    """HIP realizes a pointwise chain as one kernel: interior nodes stay unrealized
    (the reference's CPU order realizes them, csrc/tests/backend/test_runtime.cpp:42)."""
    a, b, c = (T(np.full((2, 2), v, np.float32), hip) for v in (2.0, 3.0, 4.0))
    ab = a + b
    d = ab * c
    d.realize()
    assert d._node.is_realized and not ab._node.is_realized
    assert d.numpy().tolist() == [[20, 20], [20, 20]]
    v = T(np.ones((2, 3, 4), np.float32), hip)
    r = v.reshape((6, 4)).realize()
    assert r._node.data.ptr == v._node.data.ptr  # zero-copy view


# ------------------------------------------------------- config 2: broadcast chain
def c2_inputs(rows, cols, seed=1):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (rows, cols)).astype(np.float32)
    bias = rng.normal(0, 0.1, (cols,)).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, (rows, 1)).astype(np.float32)
    return x, bias, scale


def c2(dev, x, bias, scale):
    X, B, S = T(x, dev), T(bias, dev), T(scale, dev)
    return ((X + B) * S).tanh() * X.sigmoid() - 0.1 * X * X


def c2_exact(x, bias, scale):
    """float64 value of the chain on the fp32 inputs (0.1 as the fp32 leaf the
    graph uses), and s = |p| + |q| for z = p - q: the magnitude the final
    subtraction cancels, which scales every fp32 evaluation's error."""
    x64, b64, s64 = x.astype(np.float64), bias.astype(np.float64), scale.astype(np.float64)
    p = np.tanh((x64 + b64) * s64) / (1.0 + np.exp(-x64))
    q = float(np.float32(0.1)) * x64 * x64
    return p - q, np.abs(p) + np.abs(q)


def check_c2(got, want, x, bias, scale):
    """Condition-aware parity. Every element: |got - exact| <= 16 u s (the chain's
    roundings, 3-ulp tanh and sigmoid, and the cancellation of p - q). Elements
    without cancellation (s <= 1.5 |exact|) are held to rtol 1e-6 against the
    oracle, with no absolute floor; the oracle itself meets the first bound."""
    exact, s = c2_exact(x, bias, scale)
    u = 2.0 ** -24
    assert np.all(np.abs(got.astype(np.float64) - exact) <= 16 * u * s)
    assert np.all(np.abs(want.astype(np.float64) - exact) <= 16 * u * s)
    calm = s <= 1.5 * np.abs(exact)
    assert calm.size < 4096 or calm.mean() > 0.5
    assert np.all(np.abs(got[calm] - want[calm]) <= 1e-6 * np.abs(want[calm]))


@pytest.mark.parametrize("shape", [(64, 128), (37, 129), (1, 4), (3, 1), (256, 4100)])
def test_c2_parity_small(cpu, hip, shape):
    x, bias, scale = c2_inputs(*shape)
    got = c2(hip, x, bias, scale).numpy()
    want = c2(cpu, x, bias, scale).numpy()
    check_c2(got, want, x, bias, scale)


def test_c2_full_size(cpu, hip):
    """(8192, 4096): GPU vs the oracle's fused tape on the same inputs."""
    x, bias, scale = c2_inputs(8192, 4096)
    got = c2(hip, x, bias, scale).numpy()
    want_t = c2(cpu, x, bias, scale)
    from ormi_amd import ormi_backend as ob

    ob.execute_jit(want_t._node)  # one tape over the whole chain (faster than per-node)
    want = want_t.numpy()
    check_c2(got, want, x, bias, scale)


def test_pointwise_ops_match_oracle(cpu, hip):
    rng = np.random.default_rng(21)
    a = rng.uniform(-3, 3, (33, 65)).astype(np.float32)
    b = rng.uniform(0.5, 2, (65,)).astype(np.float32)
    for name in ("exp", "sin", "cos", "tanh", "sigmoid", "gelu", "relu"):
        got = getattr(T(a, hip), name)().numpy()
        want = getattr(T(a, cpu), name)().numpy()
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6, err_msg=name)
    for dev_pair in [(hip, cpu)]:
        outs = [((T(a, d) * T(a, d) + T(b, d)) / T(b, d) - T(a, d)).numpy() for d in dev_pair]
        assert_bits_equal(outs[0], outs[1])  # + - * / without contraction: bit-exact
        outs = [(T(np.abs(a) + 0.1, d).log() + T(b, d) ** T(a, d)).numpy() for d in dev_pair]
        np.testing.assert_allclose(outs[0], outs[1], rtol=2e-6, atol=1e-6)


def _ulp_error(got, truth64):
    ulp = np.spacing(np.abs(truth64).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - truth64) / ulp


def test_device_tanh_sigmoid_accuracy(cpu, hip):
    """The device exp, tanh and sigmoid (hardware exp/rcp plus a fitted
    polynomial) stay within 2-3 ulp of float64 over dense sweeps, and within
    rtol 1e-6 of the oracle (glibc) with no absolute floor."""
    rng = np.random.default_rng(31)
    x = np.concatenate([np.linspace(-12, 12, 2_000_001, dtype=np.float32),
                        rng.standard_normal(1_000_000).astype(np.float32),
                        np.float32(0.625) + np.arange(-512, 512, dtype=np.float32) * np.float32(2 ** -24)])
    t = T(x, hip).tanh().numpy()
    assert _ulp_error(t, np.tanh(x.astype(np.float64))).max() <= 3.0
    np.testing.assert_allclose(t, T(x, cpu).tanh().numpy(), rtol=1e-6, atol=0)
    xs = np.concatenate([x, np.linspace(-80, 30, 1_000_001, dtype=np.float32)])
    s = T(xs, hip).sigmoid().numpy()
    truth = 1.0 / (1.0 + np.exp(-xs.astype(np.float64)))
    assert _ulp_error(s, truth).max() <= 3.0
    np.testing.assert_allclose(s, T(xs, cpu).sigmoid().numpy(), rtol=1e-6, atol=0)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-30, -1e-30, 200.0, -200.0], np.float32)
    ts = T(special, hip).tanh().numpy()
    assert np.array_equal(np.signbit(ts[:2]), [False, True]) and ts[0] == 0 and ts[1] == 0
    assert ts[2] == 1 and ts[3] == -1 and np.isnan(ts[4]) and ts[5] == np.float32(1e-30) and ts[7] == 1 and ts[8] == -1
    # exp: 2 ulp wherever the result is a normal float (x >= -87.3)
    xe = np.concatenate([np.linspace(-87.3, 88.7, 2_000_001, dtype=np.float32), x])
    e = T(xe, hip).exp().numpy()
    assert _ulp_error(e, np.exp(xe.astype(np.float64))).max() <= 2.0
    np.testing.assert_allclose(e, T(xe, cpu).exp().numpy(), rtol=1e-6, atol=0)
    es = T(np.array([np.inf, -np.inf, np.nan, 0.0, 89.0, -200.0], np.float32), hip).exp().numpy()
    assert es[0] == np.inf and es[1] == 0 and np.isnan(es[2]) and es[3] == 1 and es[4] == np.inf and es[5] == 0
    ss = T(special, hip).sigmoid().numpy()
    assert ss[0] == 0.5 and ss[2] == 1 and ss[3] == 0 and np.isnan(ss[4]) and ss[7] == 1 and ss[8] == 0


def test_views_and_strides_as_leaves(cpu, hip):
    rng = np.random.default_rng(22)
    x = rng.standard_normal((16, 24)).astype(np.float32)
    y = rng.standard_normal((24, 16)).astype(np.float32)
    got = (T(x, hip).transpose() * T(y, hip) + T(x, hip).reshape((24, 16))).numpy()
    want = (T(x, cpu).transpose() * T(y, cpu) + T(x, cpu).reshape((24, 16))).numpy()
    assert_bits_equal(got, want)
    e_h = T(x[:1], hip).expand((16, 24)) * T(x, hip)
    e_c = T(x[:1], cpu).expand((16, 24)) * T(x, cpu)
    assert_bits_equal(e_h.numpy(), e_c.numpy())


# Row-aligned map tiles. A tile is 256 threads x the planned unroll groups (a
# group is 4 floats when every operand allows 128-bit accesses, else 1).
# rows=1: a tile spans P whole rows (lane constants, last-dim-only operands
# loaded once, a partial last tile when P does not divide the row count);
# rows=2: a tile lies in one row; rows=3: a tile is one row; rows=0: neither;
# rows=4: rows=2 over a bias row with an even row count, the tile `unroll` rows
# of one 256-group window (the bias loaded once per lane for all of them).
def row_graph(dev, x, bias, scale, xt=None):
    X, B, S = T(x, dev), T(bias, dev), T(scale, dev)
    z = (X + B) * S - X * 0.5
    if xt is not None:  # a transposed operand: 1-float groups
        z = z + T(xt, dev).transpose().realize() * S  # the realized view aliases xt's buffer
    return z


def row_inputs(rows, cols, vec1, seed=31):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    bias = rng.normal(0, 0.1, cols).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, (rows, 1)).astype(np.float32)
    xt = rng.standard_normal((cols, rows)).astype(np.float32) if vec1 else None
    return x, bias, scale, xt


def row_case(tile, case):
    """(shape, rows mode, 1-float groups) for a tile of `tile` groups."""
    return {"span": ((33, 256), 1, False), "span_full": ((32, 256), 1, False), "span_vec1": ((33, 256), 1, True),
            "one": ((6, 4 * tile), 3, False), "one_vec1": ((5, tile), 3, True), "inside": ((3, 8 * tile), 2, False),
            "inside_vec1": ((3, 3 * tile), 2, True), "rowtile": ((4, 8 * tile), 4, False),
            "rowtile_vec1": ((2, 3 * tile), 4, True), "rowtile_nw6": ((6, 12 * tile), 4, False),
            "none": ((7, 300), 0, False)}[case]


@pytest.mark.parametrize("case", ["span", "span_full", "span_vec1", "one", "one_vec1", "inside", "inside_vec1", "rowtile",
                                  "rowtile_vec1", "rowtile_nw6", "none"])
def test_row_aligned_map_tiles(ob, cpu, hip, case):
    shape, mode, vec1 = row_case(map_tile_groups(ob), case)
    x, bias, scale, xt = row_inputs(*shape, vec1)
    z = row_graph(hip, x, bias, scale, xt)
    plan = ob._plan_kernel(z._node)["plan"]
    assert f"rows={mode}" in plan and ("vec=1" in plan) == vec1, plan
    assert_bits_equal(z.numpy(), row_graph(cpu, x, bias, scale, xt).numpy())


@pytest.mark.parametrize("mode", [1, 2, 3])
def test_row_aligned_map_tiles_3d(ob, cpu, hip, mode):
    """Three dims that do not merge: the outer coordinates come from the row
    index by division (per lane for rows=1, per tile for rows=2 and 3)."""
    tile = map_tile_groups(ob)
    c = {1: 256, 2: 8 * tile, 3: 4 * tile}[mode]
    rng = np.random.default_rng(32)
    a, b, s = (rng.standard_normal(sh).astype(np.float32) for sh in ((4, 1, c), (1, 3, c), (4, 3, 1)))

    def graph(dev):
        A, B, C = T(a, dev), T(b, dev), T(s, dev)
        return A * B + C - A / (C * C + 1.0)

    z = graph(hip)
    plan = ob._plan_kernel(z._node)["plan"]
    assert f"rows={mode}" in plan and "ndim=3" in plan, plan
    assert_bits_equal(z.numpy(), graph(cpu).numpy())


def test_row_tiles_3d(ob, cpu, hip):
    """Tiles of two rows over a bias row with three dims that do not merge: each
    row's outer coordinates come from its own index by division."""
    c = 8 * map_tile_groups(ob)
    rng = np.random.default_rng(34)
    a, s, bias = (rng.standard_normal(sh).astype(np.float32) for sh in ((4, 1, c), (4, 3, 1), (c,)))

    def graph(dev):
        A, C, B = T(a, dev), T(s, dev), T(bias, dev)
        return (A + B) * C - A / (C * C + 1.0)

    z = graph(hip)
    plan = ob._plan_kernel(z._node)["plan"]
    assert "rows=4" in plan and "ndim=3" in plan, plan
    assert_bits_equal(z.numpy(), graph(cpu).numpy())


@pytest.mark.parametrize("case", ["span", "span_vec1", "one", "inside", "rowtile", "rowtile_nw6"])
def test_row_aligned_map_tiles_grid_stride(ob, hip, case):
    """More tiles than the grid holds (64 blocks per CU), so every block walks
    several tiles and the row cursor advances with the grid stride. The chain is
    + - x only, so numpy's float32 arithmetic in the same order is the exact
    answer (the oracle's tape computes the same bits; numpy keeps the 30-70M
    element cases to seconds)."""
    tile = map_tile_groups(ob)
    grid = 256 * 64
    shape, mode, vec1 = {"span": ((grid * tile // 64 + 17, 256), 1, False),  # 64 groups a row
                         "span_vec1": ((grid * tile // 256 + 5, 256), 1, True),  # 256 groups a row
                         "one": ((grid + 16, 4 * tile), 3, False),
                         "inside": ((grid // 2 + 9, 8 * tile), 2, False),
                         "rowtile": ((grid // 2 + 8, 8 * tile), 4, False),  # 4 windows a row
                         "rowtile_nw6": ((grid // 3 + 11, 12 * tile), 4, False)}[case]  # 6 windows: grid rounded to 16380
    x, bias, scale, xt = row_inputs(*shape, vec1, seed=33)
    z = row_graph(hip, x, bias, scale, xt)
    plan = ob._plan_kernel(z._node)["plan"]
    assert f"rows={mode}" in plan, plan
    assert -(-int(plan.split("groups=")[1].split()[0]) // tile) > grid  # tiles, the last one possibly partial
    want = (x + bias) * scale - x * np.float32(0.5)
    if xt is not None:
        want = want + xt.T * scale
    assert_bits_equal(z.numpy(), want)


def test_empty_tensors_match_oracle(cpu, hip):
    """0-length dims on the HIP device: the same shapes, values and errors as
    the oracle (maps and products with nothing to compute launch nothing; sums
    over nothing fill zeros; max/argmax over nothing raise)."""
    want, got = empty_tensor_cases(cpu), empty_tensor_cases(hip)
    assert want.keys() == got.keys()
    for name in want:
        w, g = want[name], got[name]
        if isinstance(w, tuple):
            assert isinstance(g, tuple) and g[0] == "error" and "zero-size" in g[1], (name, g)
        else:
            assert not isinstance(g, tuple), (name, g)
            assert g.shape == w.shape and g.dtype == w.dtype, (name, g.shape, w.shape)
            np.testing.assert_array_equal(g, w, err_msg=name)


def test_bf16_leaves_and_casts(cpu, hip):
    rng = np.random.default_rng(23)
    x = rng.standard_normal((40, 64)).astype(np.float32)
    got = (T(x, hip, dtype="bfloat16") * 2.0 + 1.0).numpy()
    want = (T(x, cpu, dtype="bfloat16") * 2.0 + 1.0).numpy()
    assert_bits_equal(got, want)
    got = T(x, hip).astype("bfloat16").numpy()
    want = T(x, cpu).astype("bfloat16").numpy()
    assert_bits_equal(got, want)


# ---------------------------------------------------------- config 3: reductions
@pytest.fixture(scope="module")
def c3():
    return np.random.default_rng(2).normal(0, 2, (16384, 8192)).astype(np.float32)


def test_c3_row_max_and_argmax_bit_exact(cpu, hip, c3):
    xh, xc = T(c3, hip), T(c3, cpu)
    assert_bits_equal(xh.max(1).numpy(), xc.max(1).numpy())
    am = xh.argmax(1).numpy()
    assert am.dtype == np.int64
    assert_bits_equal(am, xc.argmax(1).numpy())
    assert np.array_equal(am, np.argmax(c3, axis=1))


def check_sums(got, want, x, axis):
    """Condition-aware parity of fp32 sums, kappa = sum|x| / |sum x| per output:
      * well-conditioned outputs (kappa <= 50) within rtol 1e-5 of the oracle and
        of float64, no absolute floor (the oracle's sequential order keeps its own
        error below 1e-6 relative there at these lengths);
      * outputs with kappa <= 100 within rtol 1e-5 of float64;
      * over all outputs, the HIP errors against float64 are no larger than the
        oracle's (largest and root-mean-square): the tree order is at least as
        accurate as the reference's sequential one (csrc/backend/cpu/kernels/reduce/sum.cpp:22-48);
      * every output within the Higham bound n eps sum|x|."""
    x64 = x.astype(np.float64)
    exact = x64.sum(axis=axis)
    kappa = np.abs(x64).sum(axis=axis) / np.maximum(np.abs(exact), 1e-300)
    eh = np.abs(got.astype(np.float64) - exact)
    eo = np.abs(want.astype(np.float64) - exact)
    calm = kappa <= 50
    assert calm.sum() >= 0.02 * calm.size
    assert np.all(np.abs(got[calm] - want[calm]) <= 1e-5 * np.abs(want[calm]))
    assert np.all(eh[kappa <= 100] <= 1e-5 * np.abs(exact[kappa <= 100]))
    assert eh.max() <= eo.max() and np.sqrt((eh ** 2).mean()) <= np.sqrt((eo ** 2).mean())
    assert np.all(eh <= fp32_sum_tolerance(x, axis))


def test_c3_row_sum_mean(cpu, hip, c3):
    xh, xc = T(c3, hip), T(c3, cpu)
    got = xh.sum(1).numpy()
    want = xc.sum(1).numpy()
    check_sums(got, want, c3, 1)
    # mean = sum * 2^-13 on both devices: the same checks apply to the oracle's mean
    mean_h, mean_c = xh.mean(1).numpy(), xc.mean(1).numpy()
    check_sums(mean_h * 8192, mean_c * 8192, c3, 1)
    assert np.array_equal(mean_h, got * np.float32(2 ** -13)) and np.array_equal(mean_c, want * np.float32(2 ** -13))


def test_c3_softmax_denominator(cpu, hip, c3):
    def sumexp(dev):
        x = T(c3, dev)
        return (x - x.max(1, keepdims=True)).exp().sum(1).numpy()

    got, want = sumexp(hip), sumexp(cpu)
    np.testing.assert_allclose(got, want, rtol=1e-5)


def test_c3_column_sum(cpu, hip, c3):
    got = T(c3, hip).sum(0).numpy()
    want = T(c3, cpu).sum(0).numpy()
    check_sums(got, want, c3, 0)


@pytest.mark.parametrize("shape,axes", [
    ((7, 5), (0,)), ((7, 5), (1,)), ((7, 5), None), ((3, 4, 5), (0, 2)), ((3, 4, 5), (1,)),
    ((2, 3, 4, 5), (1, 2)), ((1, 1000003), (1,)), ((1000003,), None), ((513, 3), (0,)), ((5, 1, 7), (1,)),
    # long rows, enough of them for one pass: four waves share a row (uneven pieces; 128-bit and scalar loads)
    ((4099, 4108), (1,)), ((4100, 4097), (1,)),
    # one long row in ~2,900 parts: the finish pass combines them in batches of 1,024 with a guarded tail
    ((1, 3000017), (1,)),
])
def test_reduction_shapes(cpu, hip, shape, axes):
    rng = np.random.default_rng(24)
    x = rng.integers(-8, 8, shape).astype(np.float32)  # small ints: sums are exact in fp32
    for name in ("sum", "max"):
        got = getattr(T(x, hip), name)(axes).numpy()
        want = getattr(T(x, cpu), name)(axes).numpy()
        assert_bits_equal(got, want)
    if axes is None or len(axes) == 1:
        ax = None if axes is None else axes[0]
        assert np.array_equal(T(x, hip).argmax(ax).numpy(), np.argmax(x, axis=ax))


def test_argmax_ties_and_nan(cpu, hip):
    x = np.zeros((4, 300), np.float32)
    x[0, 7] = x[0, 250] = 5.0
    x[1, :] = -np.inf
    x[2, 100] = np.nan
    x[2, 200] = np.nan
    x[3, 0] = -0.0
    for axis in (0, 1):
        got = T(x, hip).argmax(axis).numpy()
        want = T(x, cpu).argmax(axis).numpy()
        assert np.array_equal(got, want)
    assert np.array_equal(T(x, hip).argmax(1).numpy(), np.argmax(x, axis=1))
    assert_bits_equal(T(x, hip).max(1).numpy(), T(x, cpu).max(1).numpy())


@pytest.mark.parametrize("shape,axis", [((3, 1 << 20), 1), ((1 << 16, 6), 0), ((5, 1003), 1), ((1003, 70), 0),
                                        ((4099, 4108), 1), ((4100, 4097), 1)])
def test_argmax_edge_cases_all_paths(cpu, hip, shape, axis):
    """Row, column and two-pass (split) reductions, and rows that several waves
    share: the first maximum wins across lanes, vector slots, waves and parts;
    all -inf, NaN first / later, +-0 first."""
    rng = np.random.default_rng(43)
    x = rng.standard_normal(shape).astype(np.float32)
    xm = np.moveaxis(x, axis, -1)  # view: reduced axis last
    n = xm.shape[-1]
    xm[0, :] = -np.inf
    xm[1, :] = 0.0
    xm[1, 0] = -0.0                           # first zero is -0.0: max keeps its bits
    xm[1, n // 3] = -0.0
    xm[2, n - 1] = np.nan
    xm[2, n - 2] = np.nan                     # the first NaN (n-2) wins
    if xm.shape[0] > 3:
        xm[3, :] = 1.0
        xm[3, n - 5] = 7.0
        xm[3, 3] = 7.0                        # ties across the row: index 3
    for red in ("argmax", "max"):
        got = getattr(T(x, hip), red)(axis).numpy()
        want = getattr(T(x, cpu), red)(axis).numpy()
        assert_bits_equal(got, want)
    assert np.array_equal(T(x, hip).argmax(axis).numpy(), np.argmax(x, axis=axis))


# ------------------------------------------ config 1: fused pointwise + row sum
def c1_graph(dev, a, b, c):
    A, B, C = T(a, dev, requires_grad=True), T(b, dev, requires_grad=True), T(c, dev, requires_grad=True)
    y = ((A * B + C).relu() * 0.5).sum(1)
    return A, B, C, y


def test_c1_forward_backward(cpu, hip):
    rng = np.random.default_rng(0)
    a, b, c = (rng.uniform(-1, 1, (1024, 1024)).astype(np.float32) for _ in range(3))
    Ah, Bh, Ch, yh = c1_graph(hip, a, b, c)
    Ac, Bc, Cc, yc = c1_graph(cpu, a, b, c)
    got, want = yh.numpy(), yc.numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    yh.sum().backward()
    yc.sum().backward()
    for gh, gc in ((Ah.grad, Ac.grad), (Bh.grad, Bc.grad), (Ch.grad, Cc.grad)):
        assert_bits_equal(gh.numpy(), gc.numpy())  # products of exact values and a mask


def test_c1_grads_realized_together(cpu, hip):
    """realize_all puts the three gradients in one multi-output kernel; the
    results are the same bits as realizing them one by one and as the oracle."""
    from ormi_amd import realize_all

    rng = np.random.default_rng(0)
    a, b, c = (rng.uniform(-1, 1, (1024, 1024)).astype(np.float32) for _ in range(3))
    Ah, Bh, Ch, yh = c1_graph(hip, a, b, c)
    yh.sum().backward()
    grads = [Ah.grad, Bh.grad, Ch.grad]
    realize_all(*grads)
    assert all(g._node.is_realized for g in grads)
    A1, B1, C1, y1 = c1_graph(hip, a, b, c)
    y1.sum().backward()
    Ac, Bc, Cc, yc = c1_graph(cpu, a, b, c)
    yc.sum().backward()
    for g, g1, gc in zip(grads, (A1.grad, B1.grad, C1.grad), (Ac.grad, Bc.grad, Cc.grad)):
        assert_bits_equal(g.numpy(), g1.numpy())
        assert_bits_equal(g.numpy(), gc.numpy())


def test_realize_all_mixed_group(cpu, hip):
    """Mixed requests: two shapes, a reduction, a root inside another root's
    region, a duplicate, an already-realized tensor and a bf16 output."""
    from ormi_amd import realize_all

    rng = np.random.default_rng(41)
    x = rng.standard_normal((37, 130)).astype(np.float32)
    v = rng.standard_normal((130,)).astype(np.float32)

    def graph(dev):
        X, V = T(x, dev), T(v, dev)
        h = (X * V).tanh()
        return [h, h * 2.0 - X, (X + V).sigmoid().astype("bfloat16"), h.sum(1), V * V, X.max(0), h]

    got = graph(hip)
    got[4].realize()
    realize_all(*got)
    want = graph(cpu)
    for i, (g, w) in enumerate(zip(got, want)):
        assert g._node.is_realized
        gn, wn = g.numpy(), w.numpy()
        assert gn.dtype == wn.dtype and gn.shape == wn.shape
        # entry 2 is rounded to bf16: a 1-ulp fp32 difference may move it by one bf16 ulp (2^-8)
        rtol = 2 ** -8 if i == 2 else 1e-5
        np.testing.assert_allclose(gn.astype(np.float32), wn.astype(np.float32), rtol=rtol, atol=1e-5)


# ---------------------------------------------------------------- config 4: GEMM
def gemm_ref64(a, b):
    return a.astype(np.float64) @ b.astype(np.float64)


def bf16_round(x):
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("m,k,n", [(64, 64, 64), (256, 256, 256), (300, 200, 100), (33, 17, 9), (512, 1024, 768)])
def test_fp32_gemm_vs_oracle(cpu, hip, m, k, n):
    rng = np.random.default_rng(31)
    a = rng.normal(0, 1 / 8, (m, k)).astype(np.float32)
    b = rng.normal(0, 1 / 8, (k, n)).astype(np.float32)
    got = (T(a, hip) @ T(b, hip)).numpy()
    want = (T(a, cpu) @ T(b, cpu)).numpy()
    bound = 2 * k * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b))
    assert np.all(np.abs(got - want) <= bound)
    assert np.all(np.abs(got - gemm_ref64(a, b)) <= bound)


@pytest.mark.parametrize("m,k,n", [(256, 256, 256), (512, 512, 512), (300, 200, 104), (1024, 64, 2048)])
def test_bf16_gemm_vs_oracle(cpu, hip, m, k, n):
    rng = np.random.default_rng(32)
    a = rng.normal(0, 1 / 64, (m, k)).astype(np.float32)
    b = rng.normal(0, 1 / 64, (k, n)).astype(np.float32)
    got = (T(a, hip, dtype="bfloat16") @ T(b, hip, dtype="bfloat16")).numpy()
    want = (T(a, cpu, dtype="bfloat16") @ T(b, cpu, dtype="bfloat16")).numpy()
    scale = np.abs(want).max()
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=1e-3 * scale)
    exact = gemm_ref64(bf16_round(a), bf16_round(b))
    bound = 2 * k * np.finfo(np.float32).eps * (np.abs(bf16_round(a)).astype(np.float64) @ np.abs(bf16_round(b)))
    assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("k", [32, 64, 96, 128, 160, 192, 320, 2048])
def test_bf16_gemm_k_depths(hip, k):
    """Short and long K through every layout: pipelines shorter than their stage
    count, ragged M / N edges (264 x 136 is not a multiple of any tile)."""
    rng = np.random.default_rng(35 + k)
    m, n = 264, 136
    a = bf16_round(rng.normal(0, 1, (m, k)).astype(np.float32))
    b = bf16_round(rng.normal(0, 1, (k, n)).astype(np.float32))
    exact = gemm_ref64(a, b)
    bound = 2 * k * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b))
    A_n, B_n = T(a, hip, dtype="bfloat16"), T(b, hip, dtype="bfloat16")
    A_t, B_t = T(a.T.copy(), hip, dtype="bfloat16").transpose(), T(b.T.copy(), hip, dtype="bfloat16").transpose()
    for name, A, B in (("NN", A_n, B_n), ("NT", A_n, B_t), ("TN", A_t, B_n), ("TT", A_t, B_t)):
        got = (A @ B).numpy()
        assert np.all(np.abs(got - exact) <= bound), name


def test_gemm_transposed_layouts(cpu, hip):
    """NN, NT, TN, TT through transpose views: the layouts of the forward and the two
    backward GEMMs (reference csrc/core/ops/blas/matmul.cpp:86-124)."""
    rng = np.random.default_rng(33)
    a = rng.standard_normal((320, 192)).astype(np.float32)
    b = rng.standard_normal((192, 448)).astype(np.float32)
    exact = gemm_ref64(a, b)
    bound = 2 * 192 * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b))
    for dt in ("float32", "bfloat16"):
        if dt == "bfloat16":
            ar, br = bf16_round(a), bf16_round(b)
            ex = gemm_ref64(ar, br)
            bd = 2 * 192 * np.finfo(np.float32).eps * (np.abs(ar).astype(np.float64) @ np.abs(br))
        else:
            ex, bd = exact, bound
        A_n, B_n = T(a, hip, dtype=dt), T(b, hip, dtype=dt)
        A_t, B_t = T(a.T.copy(), hip, dtype=dt).transpose(), T(b.T.copy(), hip, dtype=dt).transpose()
        for A, B in ((A_n, B_n), (A_n, B_t), (A_t, B_n), (A_t, B_t)):
            got = (A @ B).numpy()
            assert np.all(np.abs(got - ex) <= bd), dt


def test_gemm_batched_broadcast(cpu, hip):
    rng = np.random.default_rng(34)
    a = rng.standard_normal((3, 2, 64, 96)).astype(np.float32)
    b = rng.standard_normal((2, 96, 32)).astype(np.float32)
    got = (T(a, hip) @ T(b, hip)).numpy()
    want = (T(a, cpu) @ T(b, cpu)).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)


def test_c4_bf16_4096_full(hip):
    """Full config: A, B ~ N(0, 1/64) in bf16, fp32 out, the default kernel at
    its config grid (256 tiles of 256x256, XCD remap), every one of the 16.8M
    outputs against the float64 product of the bf16-rounded operands: within
    2 K eps32 (|A| |B|) (fp32 accumulation of exact bf16 products) and the
    rtol 2e-2 contract of bf16 GEMM."""
    rng = np.random.default_rng(3)
    a = rng.normal(0, 1 / 64, (4096, 4096)).astype(np.float32)
    b = rng.normal(0, 1 / 64, (4096, 4096)).astype(np.float32)
    got = (T(a, hip, dtype="bfloat16") @ T(b, hip, dtype="bfloat16")).numpy()
    ar, br = bf16_round(a).astype(np.float64), bf16_round(b).astype(np.float64)
    exact = ar @ br
    assert np.isfinite(got).all()
    bound = 2 * 4096 * np.finfo(np.float32).eps * (np.abs(ar) @ np.abs(br))
    assert np.all(np.abs(got - exact) <= bound)
    np.testing.assert_allclose(got, exact, rtol=2e-2, atol=1e-3 * np.abs(exact).max())


def test_c4_fp32_forward_and_backward(cpu, hip):
    """(2048,1024)x(1024,4096) and dA = dC.B^T, dB = A^T.dC via autograd, vs float64."""
    rng = np.random.default_rng(3)
    a = rng.normal(0, 1 / 64, (2048, 1024)).astype(np.float32)
    b = rng.normal(0, 1 / 64, (1024, 4096)).astype(np.float32)
    dc = rng.normal(0, 1, (2048, 4096)).astype(np.float32)
    A, B = T(a, hip, requires_grad=True), T(b, hip, requires_grad=True)
    C = A @ B
    np.testing.assert_allclose(C.numpy(), gemm_ref64(a, b), rtol=1e-4, atol=1e-6)
    (C * T(dc, hip)).sum().backward()
    ga = A.grad.numpy()
    gb = B.grad.numpy()
    ea = dc.astype(np.float64) @ b.T.astype(np.float64)
    eb = a.T.astype(np.float64) @ dc.astype(np.float64)
    bound_a = 2 * 4096 * np.finfo(np.float32).eps * (np.abs(dc).astype(np.float64) @ np.abs(b.T))
    bound_b = 2 * 2048 * np.finfo(np.float32).eps * (np.abs(a.T).astype(np.float64) @ np.abs(dc))
    assert np.all(np.abs(ga - ea) <= bound_a)
    assert np.all(np.abs(gb - eb) <= bound_b)


# ------------------------------------------------------------- config 5: MLP step
def mlp_step(dev, X, Yt, Ws, lr=1e-3):
    ws = [T(w, dev, requires_grad=True) for w in Ws]
    h = T(X, dev)
    for i, w in enumerate(ws):
        h = h @ w
        if i < len(ws) - 1:
            h = h.gelu()
    d = h - T(Yt, dev)
    loss = (d * d).sum() * (1.0 / (X.shape[0] * Yt.shape[1]))
    loss.backward()
    new = [(w - w.grad * lr).numpy() for w in ws]
    return loss.numpy(), new


def test_mlp_step_small_vs_oracle(cpu, hip):
    rng = np.random.default_rng(4)
    dims = [64, 256, 256, 64]
    X = rng.normal(0, 1, (128, dims[0])).astype(np.float32)
    Yt = rng.normal(0, 1, (128, dims[-1])).astype(np.float32)
    Ws = [rng.uniform(-math.sqrt(6 / i), math.sqrt(6 / i), (i, o)).astype(np.float32) for i, o in zip(dims, dims[1:])]
    lh, wh = mlp_step(hip, X, Yt, Ws)
    lc, wc = mlp_step(cpu, X, Yt, Ws)
    np.testing.assert_allclose(lh, lc, rtol=1e-5)
    for a, b in zip(wh, wc):
        np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


def test_long_elementwise_chain_is_cut_into_regions(ob, hip, cabi):
    """A 3001-op chain becomes regions of at most 256 ops (a handful of cached
    kernels, not one 3001-op kernel); the result is exact."""
    import ctypes

    x = np.random.default_rng(51).standard_normal((4, 1000)).astype(np.float32)
    before = ctypes.c_uint64(0)
    cabi.ormi_hip_rtc_cache_size(ctypes.byref(before))
    y = T(x, hip)
    for _ in range(3001):
        y = -y
    got = y.numpy()
    after = ctypes.c_uint64(0)
    cabi.ormi_hip_rtc_cache_size(ctypes.byref(after))
    assert np.array_equal(got, -x)
    assert after.value - before.value <= 3


def test_deep_chain_of_graph_breakers(ob, hip):
    """Long lazy chains through reductions and matmuls realize with an explicit
    stack, and a value feeding both a reduction and later element-wise ops is
    evaluated once (a 64-op prologue cap), so the work stays linear."""
    x = np.random.default_rng(52).standard_normal((64,)).astype(np.float32)
    y = T(x, hip)
    for _ in range(2000):
        y = y - y.max()          # after the first step the max is 0: exact
    assert np.array_equal(y.numpy(), x - x.max())
    m = T(np.array(x.max(), np.float32), hip)
    X = T(x, hip)
    y = X
    for _ in range(20000):
        y = X + (y.max() - m)    # every level is x again, exactly
    assert np.array_equal(y.numpy(), x)
    eye = T(np.eye(8, dtype=np.float32), hip)
    z = T(x.reshape(8, 8), hip)
    for _ in range(5000):
        z = z @ eye
    assert np.array_equal(z.numpy(), x.reshape(8, 8))


# ------------------------------------------------------------- float16 inputs
def f16_round(x):
    return x.astype(np.float16).astype(np.float32)


def test_f16_leaves_and_casts_match_numpy(cpu, hip):
    """float16 leaves (host conversion), device casts to float16 and bfloat16
    (v_cvt_f16_f32 and the RNE bit formula) and device widening of both, over
    the sweeps that pin the oracle (tests/test_oracle_casts.py)."""
    from test_oracle_casts import bf16_nearest_f64, bf16_sweep, f16_sweep, same_bits

    x = f16_sweep()
    with np.errstate(over="ignore"):
        want = f16_round(x)
    assert same_bits(T(x, hip).astype("float16").numpy(), want)
    assert same_bits(T(x, hip, dtype="float16").numpy(), want)
    assert same_bits((T(x, hip, dtype="float16") * 1.0).numpy(), want)   # device f16 -> f32 loads
    assert same_bits(T(x, hip).astype("float16").astype("float32").numpy(), want)
    b = bf16_sweep()
    assert same_bits(T(b, hip).astype("bfloat16").numpy(), bf16_nearest_f64(b))
    assert same_bits((T(b, hip, dtype="bfloat16") * 1.0).numpy(), bf16_nearest_f64(b))
    special = np.array([np.nan, np.inf, -np.inf, -0.0, 1e6, 1e-10], np.float32)
    got = T(special, hip).astype("float16").numpy()
    assert np.isnan(got[0]) and same_bits(got[1:], np.array([np.inf, -np.inf, -0.0, np.inf, 0.0], np.float32))


def test_bf16_and_f16_kernels_of_one_structure_stay_apart(hip):
    """The same element-wise structure over an fp16 leaf, then over a bf16 leaf
    (and fp16 then bf16 outputs), in one process: each must use its own kernel.
    Both types are stored as unsigned short; a kernel cache keyed on storage
    types alone once handed the bf16 request the fp16 kernel, which read bf16
    bits as fp16. Exact ops only (x * 0.5 + 0.25 is exact for these inputs), so
    the results are compared bit for bit."""
    rng = np.random.default_rng(347)
    x = rng.uniform(-2, 2, (3, 8, 64)).astype(np.float32)
    xh, xb = f16_round(x), bf16_round(x)
    for dtype, want in (("float16", xh), ("bfloat16", xb), ("float16", xh)):
        got = (T(x, hip, dtype=dtype) * 0.5 + 0.25).numpy()
        assert np.array_equal(got, want * np.float32(0.5) + np.float32(0.25)), dtype
    y = rng.uniform(-2, 2, (3, 8, 64)).astype(np.float32)
    for dtype, rnd in (("float16", f16_round), ("bfloat16", bf16_round), ("float16", f16_round)):
        got = (T(y, hip) * 0.5).astype(dtype).numpy()
        assert np.array_equal(got, rnd(y * np.float32(0.5))), dtype


@pytest.mark.parametrize("m,k,n", [(256, 256, 256), (264, 128, 136), (300, 200, 104), (33, 17, 9), (512, 1024, 768)])
def test_f16_gemm_layouts(cpu, hip, m, k, n):
    """f16 x f16 -> fp32 (v_mfma_f32_32x32x16_f16 on the fast paths, the generic
    kernel on ragged ones) for NN, NT, TN, TT: against float64 on the
    f16-rounded inputs within 2 K eps32 |A||B|, and against the oracle."""
    rng = np.random.default_rng(36 + k)
    a = f16_round(rng.normal(0, 1, (m, k)).astype(np.float32))
    b = f16_round(rng.normal(0, 1, (k, n)).astype(np.float32))
    exact = gemm_ref64(a, b)
    bound = 2 * k * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b))
    want = (T(a, cpu, dtype="float16") @ T(b, cpu, dtype="float16")).numpy()
    assert np.all(np.abs(want - exact) <= bound)
    A_n, B_n = T(a, hip, dtype="float16"), T(b, hip, dtype="float16")
    A_t = T(a.T.copy(), hip, dtype="float16").transpose()
    B_t = T(b.T.copy(), hip, dtype="float16").transpose()
    for name, A, B in (("NN", A_n, B_n), ("NT", A_n, B_t), ("TN", A_t, B_n), ("TT", A_t, B_t)):
        got = (A @ B).numpy()
        assert np.all(np.abs(got - exact) <= bound), name
        assert np.all(np.abs(got - want) <= 2 * bound), name


def test_f16_gemm_backward_through_autograd(cpu, hip):
    """f16 leaves feeding a matmul whose gradients flow back through the casts
    (the backward GEMMs run on fp32 gradients)."""
    rng = np.random.default_rng(37)
    a = f16_round(rng.normal(0, 1 / 8, (128, 96)).astype(np.float32))
    b = f16_round(rng.normal(0, 1 / 8, (96, 160)).astype(np.float32))
    outs = []
    for dev in (hip, cpu):
        A = T(a, dev, requires_grad=True)
        B = T(b, dev, requires_grad=True)
        C = A.astype("float16") @ B.astype("float16")
        C.gelu().sum().backward()
        outs.append((C.numpy(), A.grad.numpy(), B.grad.numpy()))
    for g, w in zip(*outs):
        np.testing.assert_allclose(g, w, rtol=1e-4, atol=1e-5)


# --------------------------------------------------------------- MAX backward
@pytest.mark.parametrize("case", range(6))
def test_max_backward_is_numpy_mask(cpu, hip, case):
    """d max routes dZ to every position equal to the maximum (ties included,
    none when the maximum is NaN): bit-exact with numpy's mask and the oracle."""
    from test_oracle_casts import max_grad_cases, max_grad_numpy, run_max_grad

    x, axis, keepdims = max_grad_cases()[case]
    shape = np.max(x, axis=axis, keepdims=keepdims).shape
    w = np.random.default_rng(11 + case).uniform(0.5, 2, shape).astype(np.float32)
    got = run_max_grad(hip, x, axis, keepdims, w)
    assert_bits_equal(got, max_grad_numpy(x, axis, keepdims, w))
    assert_bits_equal(got, run_max_grad(cpu, x, axis, keepdims, w))


def test_int64_cast_to_itself_is_exact(hip):
    """argmax indices past 2^24 survive astype('int64') (a no-op), and convert to
    float32 as numpy rounds them."""
    n = (1 << 24) + 5
    x = np.zeros((1, n), np.float32)
    x[0, n - 2] = 1.0
    idx = T(x, hip).argmax(1)
    assert idx.numpy().tolist() == [n - 2]
    assert idx.astype("int64").numpy().tolist() == [n - 2]
    assert idx.astype("float32").numpy().tolist() == [float(np.float32(n - 2))]
    v = np.array([2 ** 53 + 1, -(2 ** 40) - 1], np.int64)
    assert T(v, hip, dtype="int64").astype("int64").numpy().tolist() == v.tolist()
