"""Seeded random graphs: element-wise chains over broadcast and strided views,
reductions on random axes, bf16 and fp16 leaves and casts, realized on the HIP device
and on the CPU oracle. Exact ops must agree bit for bit; the rest within fp32
rounding of the transcendentals (rtol 1e-5) and the summation-order bound."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

UNARY = ["neg", "exp", "tanh", "sigmoid", "relu", "sin", "cos", "gelu"]
BINARY = ["add", "sub", "mul", "div"]


def _graph(dev, spec):
    from ormi_amd import Tensor

    leaves = {}
    for name, arr, dtype in spec["leaves"]:
        leaves[name] = Tensor(arr, dev, dtype=dtype)
    vals = dict(leaves)
    for out, op, args in spec["ops"]:
        a = vals[args[0]]
        if op in UNARY:
            vals[out] = getattr(a, op)() if op != "neg" else -a
        elif op in BINARY:
            b = vals[args[1]]
            vals[out] = {"add": a + b, "sub": a - b, "mul": a * b, "div": a / b}[op]
        elif op == "scale":
            vals[out] = a * args[1]
        elif op == "transpose":
            vals[out] = a.transpose()
        elif op == "sum":
            vals[out] = a.sum(args[1], keepdims=args[2])
        elif op == "max":
            vals[out] = a.max(args[1], keepdims=args[2])
        elif op == "argmax":
            vals[out] = a.argmax(args[1])
        elif op == "bf16":
            vals[out] = a.astype("bfloat16")
        elif op == "f16":
            vals[out] = a.astype("float16")
    return vals[spec["ops"][-1][0]], vals


def _make_spec(seed):
    rng = np.random.default_rng(seed)
    nd = int(rng.integers(1, 4))
    shape = [int(rng.choice([1, 3, 4, 7, 16, 33, 64, 130])) for _ in range(nd)]
    leaves, names = [], []
    for i in range(int(rng.integers(2, 4))):
        # each leaf broadcasts to `shape`: some dims dropped (leading) or set to 1
        lshape = [s if rng.random() < 0.7 else 1 for s in shape]
        drop = int(rng.integers(0, nd))
        lshape = lshape[drop:] if rng.random() < 0.3 else lshape
        arr = rng.uniform(-2, 2, lshape).astype(np.float32)
        r = rng.random()
        dtype = "bfloat16" if r < 0.15 else ("float16" if r > 0.9 else None)
        leaves.append((f"L{i}", arr, dtype))
        names.append(f"L{i}")
    ops, cur = [], names[0]
    rank = {n: a.ndim for n, a, _ in leaves}  # a value's rank: the largest of its operands'
    for j in range(int(rng.integers(3, 9))):
        r = rng.random()
        out = f"v{j}"
        if r < 0.35:
            ops.append((out, str(rng.choice(UNARY)), [cur]))
            rank[out] = rank[cur]
        elif r < 0.8:
            other = str(rng.choice(names + [o for o, _, _ in ops]))
            ops.append((out, str(rng.choice(BINARY[:3])), [cur, other]))
            rank[out] = max(rank[cur], rank[other])
        else:
            ops.append((out, "scale", [cur, float(rng.uniform(-1.5, 1.5))]))
            rank[out] = rank[cur]
        cur = out
    if nd >= 2 and rng.random() < 0.3:
        ops.append(("vt", "transpose", [cur]))
        rank["vt"] = rank[cur]
        cur = "vt"
    # reduce over an axis the value has (a chain over leaves that all dropped
    # leading dims has fewer than nd)
    rk = max(rank[cur], 1)
    red = rng.random()
    if red < 0.25:
        ops.append(("r", "sum", [cur, int(rng.integers(0, rk)), bool(rng.random() < 0.5)]))
    elif red < 0.4:
        ops.append(("r", "max", [cur, int(rng.integers(0, rk)), bool(rng.random() < 0.5)]))
    elif red < 0.5:
        ops.append(("r", "argmax", [cur, int(rng.integers(0, rk))]))
    elif red < 0.6:
        ops.append(("r", "bf16" if rng.random() < 0.5 else "f16", [cur]))
    else:
        ops.append(("r", "scale", [cur, 1.0]))
    return {"leaves": leaves, "ops": ops}


@pytest.mark.parametrize("seed", range(60))
def test_random_graph_matches_oracle(cpu, hip, seed):
    spec = _make_spec(seed)
    got_t, _ = _graph(hip, spec)
    want_t, want_vals = _graph(cpu, spec)
    got, want = got_t.numpy(), want_t.numpy()
    assert got.shape == want.shape and got.dtype == want.dtype, (spec["ops"], got.shape, want.shape)
    out, last, args = spec["ops"][-1]
    if last == "argmax":
        # Transcendental rounding may reorder near-ties, so the check is that the
        # oracle's value at the device's index is the maximum (to rounding).
        x = want_vals[args[0]].numpy().astype(np.float64)
        at = np.take_along_axis(x, np.expand_dims(got, args[1]), args[1]).squeeze(args[1])
        np.testing.assert_allclose(at, x.max(args[1]), rtol=1e-4, atol=1e-4, err_msg=str(spec["ops"]))
        return
    tol = 2 ** -7 if last == "bf16" else (2 ** -10 if last == "f16" else 1e-4)
    np.testing.assert_allclose(got.astype(np.float64), want.astype(np.float64), rtol=tol, atol=tol, equal_nan=True,
                               err_msg=str(spec["ops"]))


@pytest.mark.parametrize("seed", range(40))
def test_random_matmul_matches_oracle(cpu, hip, seed):
    """Random GEMM shapes (ragged ones included) with transposed operands,
    broadcast batch dims and fp32 or bf16 inputs, against the oracle's k-ordered
    fp32 loop. Tolerance: fp32 accumulation-order bound (n eps sum|a||b|), and
    for bf16 the same on the bf16-rounded inputs the oracle also uses."""
    from ormi_amd import Tensor

    rng = np.random.default_rng(1000 + seed)
    m, k, n = (int(rng.choice([1, 7, 16, 33, 64, 100, 128, 250, 256])) for _ in range(3))
    nb = int(rng.integers(0, 3))
    batch = [int(rng.choice([1, 2, 3])) for _ in range(nb)]
    ta, tb = bool(rng.random() < 0.4), bool(rng.random() < 0.4)
    dtype = "bfloat16" if rng.random() < 0.35 else None
    a_batch = [b if rng.random() < 0.7 else 1 for b in batch]
    b_batch = [b if rng.random() < 0.7 else 1 for b in batch]
    a = rng.standard_normal(a_batch + ([k, m] if ta else [m, k])).astype(np.float32)
    b = rng.standard_normal(b_batch + ([n, k] if tb else [k, n])).astype(np.float32)

    def run(dev):
        A, B = Tensor(a, dev, dtype=dtype), Tensor(b, dev, dtype=dtype)
        if ta:
            A = A.transpose(tuple(range(nb)) + (nb + 1, nb))
        if tb:
            B = B.transpose(tuple(range(nb)) + (nb + 1, nb))
        return (A @ B).numpy()

    got, want = run(hip), run(cpu)
    assert got.shape == want.shape
    aa = np.abs(a.astype(np.float64))
    bb = np.abs(b.astype(np.float64))
    if ta:
        aa = np.swapaxes(aa, -1, -2)
    if tb:
        bb = np.swapaxes(bb, -1, -2)
    bound = (k + 2) * np.finfo(np.float32).eps * (aa @ bb)
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound + 1e-6), (m, k, n, batch, ta, tb, dtype)


ACTS = ["none", "relu", "tanh", "sigmoid", "gelu"]


def _net(dev, spec):
    """Random small network: forward, backward, SGD updates realized in a random
    order, then the weight gradients read afterwards (a gradient GEMM fused
    into an update is computed again here)."""
    from ormi_amd import Tensor

    X, Y = Tensor(spec["X"], dev), Tensor(spec["Y"], dev)
    Ws = [Tensor(w, dev, requires_grad=True) for w in spec["W"]]
    bs = [None if b is None else Tensor(b, dev, requires_grad=True) for b in spec["b"]]
    h = X
    for W, b, act in zip(Ws, bs, spec["act"]):
        h = h @ W
        if b is not None:
            h = h + b
        if act != "none":
            h = getattr(h, act)()
    if spec["loss"] == "mse":
        d = h - Y
        loss = (d * d).sum() * (1.0 / spec["X"].shape[0])
    else:
        loss = (h * Y).sum() * 0.5
    loss.backward()
    params = Ws + [b for b in bs if b is not None]
    updates = [p - p.grad * spec["lr"] for p in params]
    got = {}
    for i in spec["order"][: len(updates)]:
        got[i] = updates[i].numpy()
    out = [loss.numpy()] + [got[i] for i in range(len(updates))] + [W.grad.numpy() for W in Ws]
    loss.zero_grad_graph()
    return out


def _net_spec(seed):
    rng = np.random.default_rng(5000 + seed)
    L = int(rng.integers(1, 4))
    dims = [int(rng.choice([16, 32, 64, 96, 128, 256])) for _ in range(L + 1)]
    n = int(rng.choice([8, 33, 64, 128, 256]))
    spec = {"X": rng.standard_normal((n, dims[0])).astype(np.float32),
            "Y": rng.standard_normal((n, dims[-1])).astype(np.float32),
            "W": [(rng.standard_normal((i, o)) / np.sqrt(i)).astype(np.float32) for i, o in zip(dims, dims[1:])],
            "b": [rng.standard_normal(o).astype(np.float32) * 0.1 if rng.random() < 0.4 else None for o in dims[1:]],
            "act": [str(rng.choice(ACTS)) for _ in range(L)],
            "loss": "mse" if rng.random() < 0.6 else "dot",
            "lr": float(rng.choice([1e-3, 0.01, 0.1]))}
    nparams = L + sum(b is not None for b in spec["b"])
    spec["order"] = [int(v) for v in rng.permutation(nparams)]
    return spec


@pytest.mark.parametrize("seed", range(30))
def test_random_network_step_fused_unfused_and_oracle(ob, cpu, hip, seed):
    spec = _net_spec(seed)
    ob.set_gemm_epilogue(True)
    fused = _net(hip, spec)
    ob.set_gemm_epilogue(False)
    try:
        plain = _net(hip, spec)
    finally:
        ob.set_gemm_epilogue(True)
    for f, p in zip(fused, plain):
        assert np.array_equal(np.atleast_1d(f).view(np.uint8), np.atleast_1d(p).view(np.uint8)), (spec["act"], spec["loss"])
    want = _net(cpu, spec)
    for f, w in zip(fused, want):
        f, w = np.asarray(f, np.float64), np.asarray(w, np.float64)
        scale = max(1.0, float(np.max(np.abs(w))))
        np.testing.assert_allclose(f, w, rtol=2e-4, atol=2e-5 * scale, err_msg=str((spec["act"], spec["loss"])))
