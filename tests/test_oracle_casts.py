"""The oracle's CAST and EQ lowerings, and the MAX backward, pinned against
references that share no code or algorithm with them.

The reference has neither op (csrc/core/dtype.h:4-8, csrc/core/ops.h:4-10), so
the anchors are the mathematics and numpy:
  * float32 -> bfloat16: an exact nearest-neighbour search in float64 between the
    two bfloat16 values that bracket x (ties to the even significand, overflow
    past max + half an ulp to inf), over every bfloat16 bracket of every binade
    with the rounding-critical low halves (0, 1, just below/at/above the tie,
    all ones) plus random ones; the oracle rounds by adding a bias instead, so a
    truncating or tie-to-away mistake fails here.
  * float32 -> float16: numpy's astype(np.float16) bits over a sweep of every
    float16 bracket of every binade from underflow to overflow with the same
    critical low bits, every subnormal tie k * 2^-25, and the range ends.
  * bfloat16/float16 -> float32: all 65,536 patterns each, against numpy.
  * EQ: numpy ==, including NaN, signed zeros and infinities, under broadcast.
  * MAX backward: numpy's mask dZ * (x == max), every tied position included.
Leaf uploads with dtype= go through the binding's own host conversions, which
the same references pin.
"""
import numpy as np
import pytest


def T(data, dev="cpu", **kw):
    from ormi_amd import Tensor

    return Tensor(data, device=dev, **kw)


# -------------------------------------------------------------- test vectors
def _f32_from_bits(bits):
    return np.asarray(bits, np.uint32).view(np.float32)


def _critical_low_bits(drop_bits, rng, n_random=3):
    """Low-part patterns that decide rounding when drop_bits bits are dropped."""
    half = 1 << (drop_bits - 1)
    full = (1 << drop_bits) - 1
    pats = {0, 1, half - 1, half, half + 1, full}
    pats.update(int(v) for v in rng.integers(0, full + 1, n_random))
    return np.array(sorted(pats), np.uint32)


def bf16_sweep():
    """Every bfloat16 bracket (high 16 bits) of every binade, both signs, with
    the critical low halves: 65,536 x 9 float32 values (NaN patterns dropped)."""
    rng = np.random.default_rng(7)
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lo = _critical_low_bits(16, rng)
    bits = (hi[:, None] | lo[None, :]).reshape(-1)
    x = _f32_from_bits(bits)
    return x[~np.isnan(x)]


def f16_sweep():
    """float32 values around every float16 result: for each float32 exponent
    from 2^-27 (rounds to 0) to 2^17 (overflows), every pattern of the top 10
    significand bits with the critical low 13 bits; every subnormal tie
    (2k+1) * 2^-25; the range ends; both signs."""
    rng = np.random.default_rng(8)
    exps = np.arange(127 - 27, 127 + 18, dtype=np.uint32)
    top = np.arange(1 << 10, dtype=np.uint32) << 13
    lo = _critical_low_bits(13, rng)
    bits = (exps[:, None, None] << 23) | top[None, :, None] | lo[None, None, :]
    x = _f32_from_bits(bits.reshape(-1))
    ties = ((2 * np.arange(2048, dtype=np.float64) + 1) * 2.0 ** -25).astype(np.float32)
    ends = np.array([0.0, 2.0 ** -24, 2.0 ** -25, np.nextafter(np.float32(2.0 ** -25), np.float32(1)),
                     3 * 2.0 ** -26, 2.0 ** -14, np.nextafter(np.float32(2.0 ** -14), np.float32(0)),
                     65504.0, 65519.0, np.nextafter(np.float32(65520.0), np.float32(0)), 65520.0, 65536.0,
                     np.finfo(np.float32).max, np.inf], np.float32)
    x = np.concatenate([x, ties, ends])
    return np.concatenate([x, -x])


# ------------------------------------------------------- independent roundings
def bf16_nearest_f64(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 by exact neighbour search in
    float64 (finite inputs). Returns the float32 value of the result."""
    u = x.view(np.uint32)
    sign = (u >> 31).astype(np.uint32)
    mag = u & np.uint32(0x7FFFFFFF)
    lo_b = (mag >> 16).astype(np.int64)          # bfloat16 magnitude code below or at |x|
    hi_b = lo_b + 1                               # next code up (0x7f80 = 2^128 in an unbounded range)

    def value(code):
        e = (code >> 7) & 0xFF
        m = code & 0x7F
        v = np.where(e == 0, m / 128.0 * 2.0 ** -126, (1.0 + m / 128.0) * np.exp2(e.astype(np.float64) - 127))
        return v

    a = np.abs(x.astype(np.float64))
    d_lo, d_hi = a - value(lo_b), value(hi_b) - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((lo_b & 1) == 1))
    code = np.where(pick_hi, hi_b, lo_b)
    out = np.where(code >= 0x7F80, np.uint32(0x7F800000), (code << 16).astype(np.uint32))
    return (out | (sign << 31)).astype(np.uint32).view(np.float32)


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------------------------ bfloat16
def test_bf16_reference_rounding_is_itself_sane():
    """The neighbour search agrees with the closed-form cases it must get right."""
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, 3.3895313892515355e38,
                  3.3961775292304595e38, 2 ** -133, 2 ** -134], np.float32)
    want = np.array([1.0, 1.0, 1.0 + 2 ** -6, 1.0 + 2 ** -7, 3.3895313892515355e38, np.inf, 2 ** -133, 0.0],
                    np.float32)
    assert same_bits(bf16_nearest_f64(x), want)


def test_oracle_bf16_cast_is_rne(ob, cpu):
    x = bf16_sweep()
    want = bf16_nearest_f64(x)
    assert same_bits(T(x).astype("bfloat16").numpy(), want)
    assert same_bits(T(x, dtype="bfloat16").numpy(), want)  # the binding's host conversion


def test_oracle_bf16_cast_matches_torch(ob, cpu):
    torch = pytest.importorskip("torch")
    x = bf16_sweep()
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert same_bits(T(x).astype("bfloat16").numpy(), want)


def test_bf16_special_values(ob, cpu):
    x = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 3.4e38, -3.4e38], np.float32)
    for got in (T(x).astype("bfloat16").numpy(), T(x, dtype="bfloat16").numpy()):
        assert np.isnan(got[:2]).all()
        assert same_bits(got[2:], np.array([np.inf, -np.inf, 0.0, -0.0, np.inf, -np.inf], np.float32))


def test_bf16_widening_all_patterns(ob, cpu):
    codes = np.arange(1 << 16, dtype=np.uint32)
    want = (codes << 16).view(np.float32)
    finite = ~np.isnan(want)
    got = T(want[finite], dtype="bfloat16").numpy()   # exact values upload unchanged
    assert same_bits(got, want[finite])


# ------------------------------------------------------------------- float16
def test_oracle_f16_cast_matches_numpy(ob, cpu):
    x = f16_sweep()
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    assert same_bits(T(x).astype("float16").numpy(), want)
    assert same_bits(T(x, dtype="float16").numpy(), want)


def test_f16_special_values(ob, cpu):
    x = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1e6, -1e6, 1e-10, -1e-10], np.float32)
    for got in (T(x).astype("float16").numpy(), T(x, dtype="float16").numpy()):
        assert np.isnan(got[:2]).all()
        assert same_bits(got[2:], np.array([np.inf, -np.inf, 0.0, -0.0, np.inf, -np.inf, 0.0, -0.0], np.float32))


def test_f16_widening_all_patterns(ob, cpu):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    want = h.astype(np.float32)
    finite = ~np.isnan(want)
    assert same_bits(T(want[finite], dtype="float16").numpy(), want[finite])
    assert same_bits(T(want[finite]).astype("float16").numpy(), want[finite])


def test_cast_chain_double_rounding_order(ob, cpu):
    """bf16 -> f16 -> f32: each cast rounds once from the value it receives."""
    x = f16_sweep()
    b = bf16_nearest_f64(x)
    with np.errstate(over="ignore"):
        want = b.astype(np.float16).astype(np.float32)
    assert same_bits(T(x).astype("bfloat16").astype("float16").astype("float32").numpy(), want)


def test_cast_to_own_dtype_is_identity(ob, cpu):
    """astype to the tensor's own type keeps every value, including int64
    values that float32 cannot hold (2^24 + 1, 2^53 + 1)."""
    v = np.array([2 ** 24 + 1, -(2 ** 24) - 3, 2 ** 53 + 1, 7], np.int64)
    t = T(v, dtype="int64")
    assert t.astype("int64").numpy().tolist() == v.tolist()
    x = np.array([1.5, -2.25], np.float32)
    f = T(x)
    assert f.astype("float32")._node is f._node


# ------------------------------------------------------------------------ EQ
def test_oracle_eq_matches_numpy(ob, cpu):
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0, 1e-45, np.float32(3.4e38)], np.float32)
    a = np.repeat(specials, len(specials))
    b = np.tile(specials, len(specials))
    rng = np.random.default_rng(9)
    r = rng.integers(-3, 4, 4096).astype(np.float32)
    s = rng.integers(-3, 4, 4096).astype(np.float32)
    a, b = np.concatenate([a, r]), np.concatenate([b, s])
    node = ob.eq(T(a)._node, T(b)._node)
    ob.execute_graph(node)
    got = ob.buffer_to_numpy(node.data)
    assert got.dtype == np.float32 and same_bits(got, (a == b).astype(np.float32))
    # broadcast (rows against a column)
    m = rng.integers(0, 3, (37, 11)).astype(np.float32)
    c = rng.integers(0, 3, (37, 1)).astype(np.float32)
    node = ob.eq(T(m)._node, T(c)._node)
    ob.execute_graph(node)
    assert same_bits(ob.buffer_to_numpy(node.data), (m == c).astype(np.float32))


# -------------------------------------------------------------- MAX backward
def max_grad_cases():
    rng = np.random.default_rng(10)
    ties = rng.integers(-2, 3, (9, 13)).astype(np.float32)  # many tied maxima per row and column
    dense = rng.standard_normal((6, 7, 5)).astype(np.float32)
    nan_row = ties.copy()
    nan_row[3, 4] = np.nan
    return [(ties, 1, False), (ties, 0, True), (ties, None, False), (dense, (0, 2), False), (dense, 1, True),
            (nan_row, 1, False)]


def max_grad_numpy(x, axis, keepdims, w):
    m = np.max(x, axis=axis, keepdims=True)
    wk = w if keepdims or axis is None else np.expand_dims(w, axis)
    return (np.broadcast_to(wk, x.shape) * (x == m)).astype(np.float32)


def run_max_grad(dev, x, axis, keepdims, w):
    X = T(x, dev, requires_grad=True)
    W = T(w, dev)
    (X.max(axis, keepdims) * W).sum().backward()
    return X.grad.numpy()


@pytest.mark.parametrize("case", range(6))
def test_oracle_max_backward_is_numpy_mask(ob, cpu, case):
    x, axis, keepdims = max_grad_cases()[case]
    shape = np.max(x, axis=axis, keepdims=keepdims).shape
    w = np.random.default_rng(11 + case).uniform(0.5, 2, shape).astype(np.float32)
    got = run_max_grad(cpu, x, axis, keepdims, w)
    assert same_bits(got, max_grad_numpy(x, axis, keepdims, w))
