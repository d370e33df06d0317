"""Row reductions whose rows are shared by the four waves of a block, on random
shapes around the thresholds.

A row of at least 1024 groups of 4 elements (of 1 when rows are not 128-bit
aligned), in a reduction with enough rows that it needs no split, is cut into
four consecutive pieces of whole 64-group strides, one per wave; the waves
combine through LDS in wave order, and the launch reserves LDS so that at most
3 (sums) or 4 (max, argmax) such work-groups share a CU. Pieces are uneven
when the row length is not a multiple of 256 groups, and the last can be
short or empty.

CPU: the plans of these shapes use the shared-row kernel exactly when the row
is long enough. GPU: max and argmax bit for bit against numpy (first maximum,
NaN first), sums and means within the fp32 bound n eps32 sum|x| of float64,
on rows with planted ties across pieces, NaNs in late pieces and all -inf."""
import numpy as np
import pytest

from conftest import fp32_sum_tolerance

# (rows, cols): 128-bit rows of exactly 1024 groups, of 1027 (a short last
# piece), of 1088 (pieces of 320, 320, 320, 128), unaligned rows (scalar
# loads, 4097 and 6001 groups of 1), and a row count that is not a multiple of
# the work-groups a CU takes.
SHAPES = [(4096, 4096), (4099, 4108), (4111, 4352), (4100, 4097), (4103, 6001)]


def T(data, dev):
    from ormi_amd import Tensor

    return Tensor(data, dev)


def planted(shape, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32)
    n = shape[1]
    x[0, :] = -np.inf                                 # all -inf: index 0
    x[1, n - 3] = x[1, n - 1] = np.nan                # NaNs in the last piece: the first wins
    x[2, :] = 0.5
    x[2, 5] = x[2, n - 2] = 9.0                       # a tie across the first and last pieces
    x[3, n // 2 + 1] = 40.0                           # the maximum in a middle piece
    x[4, n - 1] = 50.0                                # the maximum at the very end
    return x


def test_plans_share_long_rows_only(ob, cpu):
    from ormi_amd import Tensor

    for rows, cols in SHAPES + [(4096, 4092)]:
        node = ob.max(Tensor(np.zeros((rows, cols), np.float32), "cpu")._node, [1], False)
        plan = ob._plan_kernel(node)["plan"]
        groups = cols // 4 if cols % 4 == 0 else cols
        assert ("waves_per_row=4" in plan) == (groups >= 1024), (rows, cols, plan)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", SHAPES)
def test_shared_rows_against_numpy(hip, shape):
    x = planted(shape, sum(shape))
    X = T(x, hip)
    got_max = X.max(1).numpy()
    got_arg = X.argmax(1).numpy()
    with np.errstate(invalid="ignore"):
        want_max = np.max(x, axis=1)
    np.testing.assert_array_equal(got_max.view(np.uint32), want_max.astype(np.float32).view(np.uint32))
    np.testing.assert_array_equal(got_arg, np.argmax(x, axis=1))

    y = x.copy()
    y[~np.isfinite(y)] = 0.0                          # sums over finite rows
    Y = T(y, hip)
    exact = y.astype(np.float64).sum(axis=1)
    bound = fp32_sum_tolerance(y, 1)
    assert np.all(np.abs(Y.sum(1).numpy().astype(np.float64) - exact) <= bound)
    mean = Y.mean(1).numpy().astype(np.float64)
    assert np.all(np.abs(mean - exact / shape[1]) <= bound / shape[1] + np.abs(exact / shape[1]) * 2 ** -23)
