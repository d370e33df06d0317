"""Element-wise kernels launched with a work-group cap.

A map over a large grid that writes at least half as many bytes as it streams
in (a copy, C2's chain, a two-input sum, a cast to bf16) is launched with an
LDS reservation it never touches, so at most 5 of its work-groups share a CU;
one that mostly reads (three inputs, one output) is not. A map on tiles of
two rows (over a bias row) takes at most 6. The reservation
changes where work-groups run, never what they compute.

CPU: which plans carry the reservation. GPU: the capped kernels bit for bit
against numpy (exact fp32 operations) and against round-to-nearest-even bf16
computed in float64."""
import numpy as np
import pytest

from test_oracle_casts import bf16_nearest_f64, same_bits

SHAPE = (8192, 4096)


def T(data, dev, **kw):
    from ormi_amd import Tensor

    return Tensor(data, dev, **kw)


def arrays(seed=11):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(SHAPE).astype(np.float32) for _ in range(3)]


def test_which_maps_are_capped(ob, cpu):
    x, y, z = arrays()
    X, Y, Z = T(x, cpu), T(y, cpu), T(z, cpu)
    capped = {"x * 2": X * 2.0, "x + y": X + Y, "x as bf16": X.astype("bfloat16")}
    for name, t in capped.items():
        assert ob._plan_kernel(t._node)["lds"] > 0, name
    assert ob._plan_kernel((X + Y + Z)._node)["lds"] == 0
    # C2's chain over a bias row: tiles of two rows, at most 6 work-groups per CU
    B, S = T(np.zeros(SHAPE[1], np.float32), cpu), T(np.ones((SHAPE[0], 1), np.float32), cpu)
    c2 = ob._plan_kernel((((X + B) * S).tanh() * X.sigmoid() - 0.1 * X * X)._node)
    assert "rows=4" in c2["plan"] and c2["lds"] == (160 * 1024 // 6 - 1024) // 512 * 512, c2["plan"]
    assert ob._plan_kernel((T(x[:256], cpu) * 2.0)._node)["lds"] == 0  # 256 work-groups: one per CU


@pytest.mark.gpu
def test_capped_maps_are_exact(hip):
    x, y, z = arrays()
    X, Y, Z = T(x, hip), T(y, hip), T(z, hip)
    assert same_bits((X * 2.0).numpy(), x * np.float32(2.0))
    assert same_bits((X + Y).numpy(), x + y)
    assert same_bits((X + Y + Z).numpy(), (x + y) + z)
    b, sc = y[0].copy(), z[:, :1].copy()  # a bias row and a per-row scale: tiles of two rows
    assert same_bits(((X + T(b, hip)) * T(sc, hip) - X).numpy(), (x + b) * sc - x)
    assert same_bits(X.astype("bfloat16").numpy(), bf16_nearest_f64(x))
    # a 64 MiB bf16 leaf: its 16-bit vector loads carry the non-temporal hint
    X16 = T(x, hip, dtype="bfloat16")
    assert same_bits((X16 * 1.0).numpy(), bf16_nearest_f64(x))


def test_bf16_leaf_of_64_mib_takes_the_load_hint(ob, cpu):
    x = arrays()[0]
    src = ob._plan_kernel((T(x, cpu, dtype="bfloat16") * 1.0)._node)["source"].split('extern "C"')[1]
    assert "__builtin_nontemporal_load((const ormi_u16x4*)" in src, src
