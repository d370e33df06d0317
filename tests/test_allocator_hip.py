"""The HIP caching allocator: size-class reuse, steady state, cache release."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_reuse_across_sizes_in_one_class(ob, hip):
    from ormi_amd import Tensor

    a = Tensor(np.ones(1000, np.float32), "hip")        # 4000 B -> 4 KiB class
    r = (a * 2.0).realize()
    s0 = ob.allocator_stats()
    del r                                                # back to the cache
    b = Tensor(np.ones(1020, np.float32), "hip")        # 4080 B: same class, reused
    s1 = ob.allocator_stats()
    assert s1["device_mallocs"] == s0["device_mallocs"]
    assert s1["reuses"] == s0["reuses"] + 1
    assert (b * 3.0).numpy().tolist() == [3.0] * 1020
    st = ob.allocator_stats()
    assert st["device_bytes"] == st["live_bytes"] + st["cached_bytes"]


def test_training_loop_reaches_steady_state(ob, hip):
    """After the first steps of a small MLP loop (forward, backward, SGD with new
    leaves each step) no step asks the device for memory. As in the reference,
    backward stores a gradient on every node and gradient graphs point back at
    forward nodes, so each step releases its graph with zero_grad_graph
    (reference csrc/core/autograd.cpp:49-58)."""
    from ormi_amd import Tensor, realize_all
    from ormi_amd.ormi_backend import Node

    rng = np.random.default_rng(4)
    X = Tensor(rng.standard_normal((64, 96)).astype(np.float32), "hip")
    Y = Tensor(rng.standard_normal((64, 32)).astype(np.float32), "hip")
    ws = [Tensor(rng.standard_normal(s).astype(np.float32) * 0.1, "hip", requires_grad=True)
          for s in ((96, 128), (128, 32))]
    mallocs = []
    for step in range(6):
        h = (X @ ws[0]).gelu() @ ws[1]
        d = h - Y
        loss = (d * d).sum() * (1.0 / d.shape[0])
        loss.backward()
        new = [w - w.grad * 1e-2 for w in ws]
        realize_all(*new)
        loss.zero_grad_graph()
        ws = [Tensor(_node=Node(n._node.data, True, n._node.device), device="hip") for n in new]
        ob.synchronize()
        mallocs.append(ob.allocator_stats()["device_mallocs"])
    assert mallocs[-1] == mallocs[-3], mallocs


def test_empty_cache_returns_cached_blocks(ob, hip):
    from ormi_amd import Tensor

    t = (Tensor(np.ones((256, 256), np.float32), "hip") + 1.0).realize()
    del t
    before = ob.allocator_stats()
    assert before["cached_bytes"] > 0
    ob.empty_cache()
    after = ob.allocator_stats()
    assert after["cached_bytes"] == 0
    assert after["device_bytes"] == after["live_bytes"]
    assert after["device_frees"] > before["device_frees"]
