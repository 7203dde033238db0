"""A whole training step of the memory layer captured in one HIP graph:
forward with routing noise (train=True; memory.py:132-226), the backward of
the queries, sub-keys and log-temperature (including the balance loss), and
the sparse value update (merge, global-norm clip, row-wise Adagrad on an
fp32 master; train.py:146-172, 378-416).  The temperature and the noise
coefficient are device scalars and no host read happens, so the step
captures; every replay from the same starting state, with eager work and
synchronisations in between, must equal the eager step bit for bit.

The captured step is built on MemoryPool.forward_backward (the forward and
backward without torch autograd), which must equal apply() followed by
torch.autograd.grad bit for bit.  The same step with torch autograd inside
the capture stays skipped: see its reason."""

import math

import pytest
import torch

from model_amd import rows as R
from model_amd.memory import MemoryPool

pytestmark = pytest.mark.gpu


@pytest.mark.skip(reason="its first run crashed the process with a segmentation fault inside "
                         "torch.cuda.CUDAGraph.capture_end (graph instantiation) after the eager step and the "
                         "warm-up had run; no cause found by reading the captured code, so the case stays off the "
                         "GPU until one is shown (the same kernels captured without torch autograd, through "
                         "MemoryPool.forward_backward, replay correctly: the tests below)")
def test_autograd_training_step_graph_replays_match_eager(gpu_lib):
    M, H, n, d_key, d, k = 2048, 4, 512, 256, 256, 16
    pool = MemoryPool(n, H, d_key, d, k, routing_noise=1.0, values_dtype=torch.float16)
    g = torch.Generator(device="cuda").manual_seed(30)
    keys0 = torch.randn((H, 2, n, d_key // 2), generator=g, device="cuda") * (d_key // 2) ** -0.5
    values0 = torch.empty((n * n, d), dtype=torch.float16, device="cuda").normal_(0.0, 0.02, generator=g)
    q0 = torch.randn((M, H, d_key), generator=g, device="cuda")
    g_out = torch.randn((M, d), generator=g, device="cuda") * 1e-3
    g_bal = torch.full((), 0.01, device="cuda")
    noise_scale = torch.full((), 0.8, device="cuda")  # annealed, as a device scalar (train.py:56-63)

    # static state the graph works on
    keys = keys0.clone().requires_grad_(True)
    log_t = torch.tensor(math.log(12.0), device="cuda", requires_grad=True)
    q = q0.clone().requires_grad_(True)
    values = values0.clone()
    upd = R.SparseRowUpdate(values, lr=1e-3, pool_lr_mult=3.0, warmup_steps=0, steps=1000, grad_clip=1.0)
    acc0, master0 = upd.acc.clone(), upd.master.clone()

    def reset():
        with torch.no_grad():
            keys.copy_(keys0)
            log_t.fill_(math.log(12.0))
            q.copy_(q0)
            values.copy_(values0)
            upd.acc.copy_(acc0)
            upd.master.copy_(master0)
        upd.step = 0

    def step():
        out, aux = pool.apply({"params": {"sub_keys": keys, "values": values, "log_temperature": log_t}}, q,
                              train=True, sparse_grad=True, noise_scale=noise_scale, rngs={"routing": 5})
        gq, gk, gt = torch.autograd.grad([out, aux["balance_loss"]], [q, keys, log_t], grad_outputs=[g_out, g_bal])
        rest = R.sum_squares([gk, gt])  # fixed order, no memset node in the graph
        upd({"slots": [aux["slots"]], "weights": [aux["weights"]]}, {0: g_out}, [0], rest_sq=rest)
        return gq, gk, gt

    reset()
    want = [t.clone() for t in step()] + [values.clone(), upd.acc.clone(), upd.master.clone()]
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            reset()
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    reset()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    names = ("d_queries", "d_sub_keys", "d_log_temperature", "values", "acc", "master")
    for i in range(3):
        reset()
        graph.replay()
        torch.cuda.synchronize()
        got = list(outs) + [values, upd.acc, upd.master]
        for name, a, b in zip(names, got, want):
            assert torch.equal(a, b), (i, name)
        assert not torch.equal(values, values0)  # the step did update rows
        torch.randn(4096, device="cuda").sum().item()  # unrelated eager work between replays



def _setup():
    M, H, n, d_key, d, k = 2048, 4, 512, 256, 256, 16
    pool = MemoryPool(n, H, d_key, d, k, routing_noise=1.0, values_dtype=torch.float16)
    g = torch.Generator(device="cuda").manual_seed(30)
    keys0 = torch.randn((H, 2, n, d_key // 2), generator=g, device="cuda") * (d_key // 2) ** -0.5
    values0 = torch.empty((n * n, d), dtype=torch.float16, device="cuda").normal_(0.0, 0.02, generator=g)
    q0 = torch.randn((M, H, d_key), generator=g, device="cuda")
    g_out = torch.randn((M, d), generator=g, device="cuda") * 1e-3
    return pool, keys0, values0, q0, g_out


def test_forward_backward_equals_autograd(gpu_lib):
    pool, keys0, values0, q0, g_out = _setup()
    g_bal = torch.full((), 0.01, device="cuda")
    noise_scale = torch.full((), 0.8, device="cuda")
    keys = keys0.clone().requires_grad_(True)
    log_t = torch.tensor(math.log(12.0), device="cuda", requires_grad=True)
    q = q0.clone().requires_grad_(True)
    params = {"sub_keys": keys, "values": values0, "log_temperature": log_t}
    out_a, aux_a = pool.apply({"params": params}, q, train=True, sparse_grad=True, noise_scale=noise_scale,
                              rngs={"routing": 5})
    ga = torch.autograd.grad([out_a, aux_a["balance_loss"]], [q, keys, log_t], grad_outputs=[g_out, g_bal])
    out_m, aux_m, gm = pool.forward_backward({"params": params}, q.detach(), g_out, g_bal, train=True,
                                             noise_scale=noise_scale, rngs={"routing": 5})
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_m)
    assert torch.equal(aux_a["slots"], aux_m["slots"]) and torch.equal(aux_a["weights"], aux_m["weights"])
    assert torch.equal(aux_a["balance_loss"], aux_m["balance_loss"])
    for name, a, b in zip(("d_queries", "d_sub_keys", "d_log_temperature"), ga, gm):
        assert a.shape == b.shape and a.dtype == b.dtype, name
        assert torch.equal(a, b), name


def test_training_step_graph_replays_match_eager(gpu_lib):
    pool, keys0, values0, q0, g_out = _setup()
    g_bal = torch.full((), 0.01, device="cuda")
    noise_scale = torch.full((), 0.8, device="cuda")  # annealed, as a device scalar (train.py:56-63)
    keys = keys0.clone()
    log_t = torch.tensor(math.log(12.0), device="cuda")
    q = q0.clone()
    values = values0.clone()
    upd = R.SparseRowUpdate(values, lr=1e-3, pool_lr_mult=3.0, warmup_steps=0, steps=1000, grad_clip=1.0)
    acc0, master0 = upd.acc.clone(), upd.master.clone()

    def reset():
        keys.copy_(keys0)
        log_t.fill_(math.log(12.0))
        q.copy_(q0)
        values.copy_(values0)
        upd.acc.copy_(acc0)
        upd.master.copy_(master0)
        upd.step = 0

    def step():
        params = {"sub_keys": keys, "values": values, "log_temperature": log_t}
        out, aux, (gq, gk, gt) = pool.forward_backward({"params": params}, q, g_out, g_bal, train=True,
                                                       noise_scale=noise_scale, rngs={"routing": 5})
        rest = R.sum_squares([gk, gt])  # fixed order, no memset node in the graph
        upd({"slots": [aux["slots"]], "weights": [aux["weights"]]}, {0: g_out}, [0], rest_sq=rest)
        return out, gq, gk, gt

    reset()
    want = [t.clone() for t in step()] + [values.clone(), upd.acc.clone(), upd.master.clone()]
    torch.cuda.synchronize()
    print("eager step done", flush=True)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            reset()
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    print("warm-up on a side stream done", flush=True)
    reset()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    print("captured", flush=True)
    names = ("out", "d_queries", "d_sub_keys", "d_log_temperature", "values", "acc", "master")
    for i in range(3):
        reset()
        graph.replay()
        torch.cuda.synchronize()
        got = list(outs) + [values, upd.acc, upd.master]
        for name, a, b in zip(names, got, want):
            assert torch.equal(a, b), (i, name)
        assert not torch.equal(values, values0)  # the step did update rows
        torch.randn(4096, device="cuda").sum().item()  # unrelated eager work between replays
        print("replay", i, "equal", flush=True)


def test_overlapped_training_step_graph_matches_serial_eager(gpu_lib):
    """The step as the training bench runs it: the sparse row merge started
    on a second stream from forward_backward's on_forward hook, the clean
    stage-1 lists on the pool's own second stream, the key diversity term
    inside the call and the dense gradients in the clip's pass; captured in
    one graph, every replay equals the same step run eagerly on one stream
    (SparseRowUpdate's __call__), bit for bit."""
    pool, keys0, values0, q0, g_out = _setup()
    g_bal = torch.full((), 0.01, device="cuda")
    g_div = torch.full((), 0.01, device="cuda")
    keys = keys0.clone()
    log_t = torch.tensor(math.log(12.0), device="cuda")
    values = values0.clone()
    upd = R.SparseRowUpdate(values, lr=1e-3, pool_lr_mult=3.0, warmup_steps=0, steps=1000, grad_clip=1.0)
    acc0, master0 = upd.acc.clone(), upd.master.clone()
    params = {"sub_keys": keys, "values": values, "log_temperature": log_t}
    merge_stream = torch.cuda.Stream()

    def reset():
        values.copy_(values0)
        upd.acc.copy_(acc0)
        upd.master.copy_(master0)
        upd.step = 0

    def serial():
        out, aux, (gq, gk, gt) = pool.forward_backward({"params": params}, q0, g_out, g_bal, train=True,
                                                       rngs={"routing": 5}, g_diversity=g_div)
        r = upd({"slots": [aux["slots"]], "weights": [aux["weights"]]}, {0: g_out}, [0], dense_grads=[gk, gt],
                count_slots=True)
        return out, gq, gk, gt, r["slot_counts"]

    def overlapped():
        cur = torch.cuda.current_stream()
        pending = {}

        def start(aux):
            merge_stream.wait_stream(cur)
            with torch.cuda.stream(merge_stream):
                pending["m"] = upd.merge({"slots": [aux["slots"]], "weights": [aux["weights"]]}, {0: g_out}, [0],
                                         count_slots=True)

        out, aux, (gq, gk, gt) = pool.forward_backward({"params": params}, q0, g_out, g_bal, train=True,
                                                       rngs={"routing": 5}, g_diversity=g_div, on_forward=start)
        cur.wait_stream(merge_stream)
        r = upd.apply(pending["m"], dense_grads=[gk, gt])
        return out, gq, gk, gt, r["slot_counts"]

    reset()
    want = [t.clone() for t in serial()] + [values.clone(), upd.acc.clone(), upd.master.clone()]
    torch.cuda.synchronize()
    reset()
    got_eager = [t.clone() for t in overlapped()] + [values.clone(), upd.acc.clone(), upd.master.clone()]
    torch.cuda.synchronize()
    names = ("out", "d_queries", "d_sub_keys", "d_log_temperature", "slot_counts", "values", "acc", "master")
    for name, a, b in zip(names, got_eager, want):
        assert torch.equal(a, b), ("eager overlapped", name)
    print("eager overlapped step equal", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            reset()
            overlapped()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    reset()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = overlapped()
    print("captured", flush=True)
    for i in range(3):
        reset()
        graph.replay()
        torch.cuda.synchronize()
        got = list(outs) + [values, upd.acc, upd.master]
        for name, a, b in zip(names, got, want):
            assert torch.equal(a, b), (i, name)
        torch.randn(4096, device="cuda").sum().item()  # unrelated eager work between replays
        print("replay", i, "equal", flush=True)


def _graph_node_types(graph):
    """Node types of a captured graph (keep_graph=True), read through the
    HIP runtime's hipGraphGetNodes / hipGraphNodeGetType."""
    import ctypes as C

    hip = C.CDLL("libamdhip64.so")
    g = C.c_void_p(int(graph.raw_cuda_graph()))
    n = C.c_size_t(0)
    assert hip.hipGraphGetNodes(g, None, C.byref(n)) == 0
    nodes = (C.c_void_p * n.value)()
    assert hip.hipGraphGetNodes(g, nodes, C.byref(n)) == 0
    types = []
    for i in range(n.value):
        t = C.c_int(-1)
        assert hip.hipGraphNodeGetType(C.c_void_p(nodes[i]), C.byref(t)) == 0
        types.append(t.value)
    return types


def test_captured_training_step_has_no_memset_nodes(gpu_lib):
    """The captured step (forward with noise, backward, the dense gradients'
    norm, merge, clip, Adagrad) records no memset node, which has given wrong
    results on replays after the first on these GPUs.  The graph still
    replays to the eager result."""
    pool, keys0, values0, q0, g_out = _setup()
    g_bal = torch.full((), 0.01, device="cuda")
    keys, values = keys0.clone(), values0.clone()
    log_t = torch.tensor(math.log(12.0), device="cuda")
    upd = R.SparseRowUpdate(values, lr=1e-3, pool_lr_mult=3.0, warmup_steps=0, steps=1000, grad_clip=1.0)
    acc0, master0 = upd.acc.clone(), upd.master.clone()

    def reset():
        keys.copy_(keys0)
        values.copy_(values0)
        upd.acc.copy_(acc0)
        upd.master.copy_(master0)
        upd.step = 0

    def step():
        params = {"sub_keys": keys, "values": values, "log_temperature": log_t}
        out, aux, (gq, gk, gt) = pool.forward_backward({"params": params}, q0, g_out, g_bal, train=True,
                                                       rngs={"routing": 9})
        rest = R.sum_squares([gk, gt])
        upd({"slots": [aux["slots"]], "weights": [aux["weights"]]}, {0: g_out}, [0], rest_sq=rest)
        return out, gk

    reset()
    want = [t.clone() for t in step()] + [values.clone()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        reset()
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    reset()
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph):
        outs = step()
    types = _graph_node_types(graph)
    print("graph nodes by type:", {t: types.count(t) for t in set(types)}, flush=True)
    assert types.count(0) > 20  # kernel nodes
    assert types.count(2) == 0, "memset node in the captured step"
    graph.instantiate()
    for i in range(2):
        reset()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "d_sub_keys", "values"), list(outs) + [values], want):
            assert torch.equal(a, b), (i, name)
