"""Evaluates the known-answer vectors of tests/golden/reference_kats.json on a
device. A case names its inputs (values, shape, optional strides and
requires_grad) and a nested expression ["op", operand, ...] over them; the
result must equal "expect" (exactly, or within the case's "atol"), or, for a
backward case, the gradients must equal "grads"."""
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_kats.json"


def cases():
    return json.loads(GOLDEN.read_text())["cases"]


def _leaf(ob, spec, dev_enum):
    arr = np.array(spec["values"], np.float32)
    buf = ob.numpy_to_buffer(arr, dev_enum)
    node = ob.Node(buf, bool(spec.get("requires_grad", False)), ob.Device(dev_enum, 0))
    shape = list(spec["shape"])
    if "strides" in spec:
        node.view = ob.TensorView(shape, list(spec["strides"]))
    else:
        node.view = ob.TensorView(shape, list(ob.calc_contiguous_strides(shape)))
    return node


def _build(ob, expr, leaves):
    if isinstance(expr, str):
        return leaves[expr]
    op, *args = expr
    if op in ("add", "sub", "mul", "div", "pow", "matmul"):
        return getattr(ob, op)(_build(ob, args[0], leaves), _build(ob, args[1], leaves))
    if op in ("neg", "exp", "sin", "cos", "log"):
        return getattr(ob, op)(_build(ob, args[0], leaves))
    if op == "sum":
        return ob.sum(_build(ob, args[0], leaves), list(args[1]), bool(args[2]))
    if op == "reshape":
        return ob.reshape(_build(ob, args[0], leaves), list(args[1]))
    if op == "transpose":
        x = _build(ob, args[0], leaves)
        return ob.transpose(x, list(reversed(range(len(x.shape)))))
    raise ValueError(f"unknown KAT op {op}")


def run_case(ob, case, dev_enum):
    leaves = {k: _leaf(ob, v, dev_enum) for k, v in case["inputs"].items()}
    root = _build(ob, case["expr"], leaves)
    if "grads" in case:
        ob.compute_gradients(root)
        for name, want in case["grads"].items():
            g = leaves[name].grad
            ob.execute_graph(g)
            got = ob.buffer_to_numpy(g.data).reshape(-1)
            assert got.tolist() == [float(v) for v in want], (case["name"], name, got)
        return
    ob.execute_graph(root)
    exp = case["expect"]
    assert list(root.shape) == list(exp["shape"]), (case["name"], root.shape)
    got = ob.buffer_to_numpy(root.data)
    strides = list(root.view.strides)
    n = int(np.prod(exp["shape"])) if exp["shape"] else 1
    # Gather the logical elements through the view (a realized view may alias).
    idx = np.indices(exp["shape"]).reshape(len(exp["shape"]), -1) if exp["shape"] else np.zeros((0, 1), int)
    off = (idx * np.array(strides)[:, None]).sum(0) if exp["shape"] else np.zeros(1, int)
    vals = got.reshape(-1)[off][:n]
    want = np.array(exp["values"], np.float32)
    atol = case.get("atol")
    if atol is None:
        assert vals.tolist() == want.tolist(), (case["name"], vals)
    else:
        assert np.allclose(vals, want, atol=atol, rtol=0), (case["name"], vals)
