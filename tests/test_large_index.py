"""Tensors past 2^31 elements: the 64-bit index paths of the generated map and
reduction kernels and the GEMM's 64-bit operand offsets (the layout sized for
288 GB of HBM). The operand is y[i, j] = (j mod 3) + (i mod 2) over 65537 x
32768 = 2^31 + 32768 elements (8.6 GB fp32). Every value is a small integer,
so every sum below is exact in fp32 whatever the order, and each result is
checked bit-exact against an integer closed form (the oracle cannot hold an
8.6 GB operand in a test's time).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

R, C = 65537, 32768  # R * C > 2^31


def T(data, dev, **kw):
    from ormi_amd import Tensor

    return Tensor(data, device=dev, **kw)


def pattern(hip):
    a = (np.arange(C) % 3).astype(np.float32)
    b = (np.arange(R) % 2).astype(np.float32).reshape(R, 1)
    return T(b, hip) + T(a, hip), a.astype(np.int64), b.reshape(R).astype(np.int64)


def test_plan_uses_64_bit_indices(ob, hip):
    y, _, _ = pattern(hip)
    assert R * C > 2**31
    assert "idx=64" in ob._plan_kernel(y._node)["plan"]


@pytest.mark.parametrize("realize_first", [False, True])
def test_row_and_column_reductions_past_2_31(hip, realize_first):
    y, a, b = pattern(hip)
    if realize_first:
        y = y.realize()  # the map kernel writes all 8.6 GB
    row_sum = y.sum(1).numpy()
    np.testing.assert_array_equal(row_sum.astype(np.int64), a.sum() + C * b)
    row_max = y.max(1).numpy()
    np.testing.assert_array_equal(row_max.astype(np.int64), 2 + b)
    row_arg = y.argmax(1).numpy()
    np.testing.assert_array_equal(row_arg, np.full(R, 2))  # first j with j mod 3 == 2
    col_sum = y.sum(0).numpy()
    np.testing.assert_array_equal(col_sum.astype(np.int64), R * a + b.sum())
    col_arg = y.argmax(0).numpy()
    np.testing.assert_array_equal(col_arg, np.full(C, 1))  # first i with i mod 2 == 1


def test_gemm_operand_past_2_31(hip):
    """A (R x C, 64-bit element offsets) times a 0/1 matrix: fp32 and bf16."""
    y, a, b = pattern(hip)
    y = y.realize()
    rng = np.random.default_rng(81)
    Bm = rng.integers(0, 2, (C, 64)).astype(np.float32)
    want = (a @ Bm.astype(np.int64))[None, :] + b[:, None] * Bm.astype(np.int64).sum(0)[None, :]
    got = (y @ T(Bm, hip)).numpy()
    np.testing.assert_array_equal(got.astype(np.int64), want)
    yb = y.astype("bfloat16")  # a cast kernel over 2^31 + 32768 elements
    got_b = (yb @ T(Bm, hip).astype("bfloat16")).numpy()
    np.testing.assert_array_equal(got_b.astype(np.int64), want)
