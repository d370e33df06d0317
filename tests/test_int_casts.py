"""Conversions between float32 and the integer dtypes (int64, int32, bool),
pinned by closed forms in exact Python integer arithmetic.

The reference declares Int32 and Bool (csrc/core/dtype.h:4-8) but computes only
in float, so it fixes no rule for converting; this build's rule is:
  * float32 -> int64 / int32: truncation toward zero; NaN gives 0; a value at
    or past the type's range saturates to its end (Python's int() of a float
    truncates exactly, and Python compares floats with ints exactly);
  * float32 -> bool: x != 0, so NaN gives true and -0.0 false;
  * int64 / int32 -> float32: round to nearest, ties to even, computed here
    from the integer's bits (no float arithmetic, so no double rounding);
  * bool -> float32: 0 or 1;
  * graph-path casts between integer types pass through float32, as every
    element-wise value does (the store of the load).
The vectors hit what decides each rule: the saturation boundaries and their
float32 neighbours, halves and near-integers, NaN, infinities, signed zeros,
and, for the int -> float direction, every binade from 2^24 to 2^62 with the
rounding-critical low bits (exact, just below, at and above the tie, on an
even and an odd kept significand). CPU: the oracle against the closed forms,
and checks that the vectors tell the right rule from a wrong one. GPU: the HIP
graph path bit for bit against the oracle, and the C-ABI ormi_hip_convert
against the closed forms (exact between integer types)."""
import ctypes

import numpy as np
import pytest

I64 = (-(1 << 63), (1 << 63) - 1)
I32 = (-(1 << 31), (1 << 31) - 1)


# ------------------------------------------------------------- closed forms
def trunc_sat(x: float, lo: int, hi: int) -> int:
    if x != x:
        return 0
    if x >= hi + 1:
        return hi
    if x <= lo:
        return lo
    return int(x)


def int_to_f32_rne(v: int) -> float:
    """The float32 nearest to the integer v, ties to an even significand."""
    if v == 0:
        return 0.0
    a = abs(v)
    n = a.bit_length()
    if n <= 24:
        q, shift = a, 0
    else:
        shift = n - 24
        q, r = divmod(a, 1 << shift)
        half = 1 << (shift - 1)
        if r > half or (r == half and q & 1):
            q += 1
    return float(-(q << shift) if v < 0 else q << shift)


# ------------------------------------------------------------------ vectors
def float_vectors() -> np.ndarray:
    f = np.float32
    vals = [0.0, -0.0, 0.5, -0.5, 0.99999994, -0.99999994, 1.0, -1.0, 1.5, -1.5, 2.5, -2.5, 3.5, -3.5,
            np.nan, -np.nan, np.inf, -np.inf, np.finfo(f).max, -np.finfo(f).max, np.finfo(f).tiny, 1e-45]
    for e in list(range(20, 66)):
        for s in (1.0, -1.0):
            p = f(s * 2.0 ** e)
            vals += [p, np.nextafter(p, f(0)), np.nextafter(p, f(s * np.inf))]
    rng = np.random.default_rng(11)
    mags = 10.0 ** rng.uniform(-3, 20, 2000)
    vals += list(mags * rng.choice([-1.0, 1.0], 2000))
    vals += list(rng.uniform(-4, 4, 500))
    return np.array(vals, np.float32)


def int_vectors(bits: int) -> np.ndarray:
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    vals = {0, 1, -1, 2, -2, lo, hi, lo + 1, hi - 1}
    for k in range(23, bits - 1):
        shift = max(k - 23, 0)
        half = 1 << (shift - 1) if shift else 0
        for low in {0, 1, max(half - 1, 0), half, half + 1, (1 << shift) - 1, (1 << shift) + half}:
            for odd in (0, 1 << shift):  # kept significand even, then odd
                v = (1 << k) + odd + low
                if v <= hi:
                    vals.update({v, -v})
    rng = np.random.default_rng(12)
    vals.update(int(x) for x in rng.integers(lo, hi, 2000, dtype=np.int64))
    return np.array(sorted(vals), np.int64 if bits == 64 else np.int32)


def expect_f2i(x: np.ndarray, dtype) -> np.ndarray:
    lo, hi = I64 if dtype == np.int64 else I32
    return np.array([trunc_sat(float(v), lo, hi) for v in x], dtype)


def expect_i2f(v: np.ndarray) -> np.ndarray:
    return np.array([int_to_f32_rne(int(x)) for x in v], np.float32)


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def T(data, dev, **kw):
    from ormi_amd import Tensor

    return Tensor(data, dev, **kw)


# ------------------------------------------------------ the vectors decide --
def test_vectors_tell_the_rules_apart():
    """A plausible wrong rule fails on these vectors: numpy's own casts (NaN
    and overflow to the minimum integer), wrapping instead of saturating at
    32 bits, truncating or rounding ties away in int -> float."""
    x = float_vectors()
    with np.errstate(invalid="ignore"):
        assert not np.array_equal(x.astype(np.int64), expect_f2i(x, np.int64))
        assert not np.array_equal(x.astype(np.int32), expect_f2i(x, np.int32))
    wrapped = np.array([int(np.int64(v)) & 0xFFFFFFFF for v in expect_f2i(x, np.int64)], np.uint32).view(np.int32)
    assert not np.array_equal(wrapped, expect_f2i(x, np.int32))
    v = int_vectors(64)
    rne = expect_i2f(v)

    def int_to_f32_trunc(x: int) -> float:
        a = abs(x)
        shift = max(a.bit_length() - 24, 0)
        return float(-(a >> shift << shift) if x < 0 else a >> shift << shift)

    assert not np.array_equal(rne, np.array([int_to_f32_trunc(int(x)) for x in v], np.float32))
    # ties away from zero: the first tie on an even significand rounds down under RNE
    k = 30
    tie = (1 << k) + (1 << (k - 24))
    assert int_to_f32_rne(tie) == float(1 << k) and int_to_f32_rne(tie + (1 << (k - 23))) == float((1 << k) + (1 << (k - 22)))
    # the closed form agrees with numpy's int -> float32 where that is a single rounding (|v| < 2^53 via float64 exact)
    small = v[np.abs(v) < (1 << 53)]
    assert np.array_equal(expect_i2f(small), small.astype(np.float64).astype(np.float32))


# ------------------------------------------------------------------ oracle --
@pytest.mark.parametrize("dtype", ["int64", "int32"])
def test_oracle_float_to_int_is_saturating_truncation(cpu, dtype):
    x = float_vectors()
    got = T(x, cpu).astype(dtype).numpy()
    assert bits_equal(got, expect_f2i(x, np.int64 if dtype == "int64" else np.int32))


def test_oracle_float_to_bool(cpu):
    x = float_vectors()
    got = T(x, cpu).astype("bool").numpy()
    assert bits_equal(got, x != 0)
    assert got[np.isnan(x)].all() and not got[(x == 0)].any()


@pytest.mark.parametrize("bits", [64, 32])
def test_oracle_int_to_float_is_rne(cpu, bits):
    v = int_vectors(bits)
    got = T(v, cpu, dtype=f"int{bits}").astype("float32").numpy()
    assert bits_equal(got, expect_i2f(v))
    # the same value read as an operand of arithmetic
    assert bits_equal((T(v, cpu, dtype=f"int{bits}") * 1.0).numpy(), expect_i2f(v))


def test_oracle_bool_to_float(cpu):
    b = np.array([True, False, True, True, False])
    assert bits_equal(T(b, cpu, dtype="bool").astype("float32").numpy(), b.astype(np.float32))


def test_oracle_int_to_int_goes_through_float32(cpu):
    v = int_vectors(64)
    got = T(v, cpu, dtype="int64").astype("int32").numpy()
    want = np.array([trunc_sat(int_to_f32_rne(int(x)), *I32) for x in v], np.int32)
    assert bits_equal(got, want)


# --------------------------------------------------------------------- HIP --
@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["int64", "int32", "bool"])
def test_hip_float_to_int_matches_oracle(cpu, hip, dtype):
    x = float_vectors()
    got = T(x, hip).astype(dtype).numpy()
    assert bits_equal(got, T(x, cpu).astype(dtype).numpy())
    # fused with arithmetic: the store of a computed value
    y = (T(x, hip) * 1.0 + 0.0).astype(dtype).numpy()
    assert bits_equal(y, (T(x, cpu) * 1.0 + 0.0).astype(dtype).numpy())


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [64, 32])
def test_hip_int_to_float_matches_oracle(cpu, hip, bits):
    v = int_vectors(bits)
    dt = f"int{bits}"
    assert bits_equal(T(v, hip, dtype=dt).astype("float32").numpy(), expect_i2f(v))
    assert bits_equal((T(v, hip, dtype=dt) * 1.0).numpy(), expect_i2f(v))
    assert bits_equal(T(v, hip, dtype=dt).astype("int32").numpy(), T(v, cpu, dtype=dt).astype("int32").numpy())
    b = np.array([True, False, True, True, False] * 50)
    assert bits_equal(T(b, hip, dtype="bool").astype("float32").numpy(), b.astype(np.float32))


@pytest.mark.gpu
def test_hip_convert_entry_against_closed_forms(cabi, hip):
    """ormi_hip_convert: float -> integers by the closed forms, integers ->
    float32 by exact RNE, and exact conversions between integer types."""
    F32, I32c, BOOL, I64c = 0, 1, 2, 5
    size = {F32: 4, I32c: 4, BOOL: 1, I64c: 8}
    np_t = {F32: np.float32, I32c: np.int32, BOOL: np.bool_, I64c: np.int64}

    def convert(src: np.ndarray, s_dt: int, d_dt: int) -> np.ndarray:
        n = src.size
        ps, pd = ctypes.c_void_p(), ctypes.c_void_p()
        assert cabi.ormi_hip_malloc(ctypes.byref(ps), max(src.nbytes, 8)) == 0
        assert cabi.ormi_hip_malloc(ctypes.byref(pd), max(n * size[d_dt], 8)) == 0
        try:
            assert cabi.ormi_hip_memcpy_h2d(ps, src.ctypes.data, src.nbytes) == 0
            assert cabi.ormi_hip_convert(pd, d_dt, ps, s_dt, n) == 0, cabi.ormi_hip_last_error()
            out = np.empty(n, np_t[d_dt])
            assert cabi.ormi_hip_memcpy_d2h(out.ctypes.data, pd, out.nbytes) == 0
            return out
        finally:
            cabi.ormi_hip_free(ps)
            cabi.ormi_hip_free(pd)

    x = float_vectors()
    assert bits_equal(convert(x, F32, I64c), expect_f2i(x, np.int64))
    assert bits_equal(convert(x, F32, I32c), expect_f2i(x, np.int32))
    assert bits_equal(convert(x, F32, BOOL), x != 0)
    v64, v32 = int_vectors(64), int_vectors(32)
    assert bits_equal(convert(v64, I64c, F32), expect_i2f(v64))
    assert bits_equal(convert(v32, I32c, F32), expect_i2f(v32))
    assert bits_equal(convert(v64, I64c, I64c), v64)
    assert bits_equal(convert(v32, I32c, I64c), v32.astype(np.int64))
    assert bits_equal(convert(v64, I64c, I32c), np.clip(v64, *I32).astype(np.int32))
    assert bits_equal(convert(v64, I64c, BOOL), v64 != 0)
    b = np.array([True, False, True], np.bool_)
    assert bits_equal(convert(b, BOOL, I64c), b.astype(np.int64))
