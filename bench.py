"""Benchmark of the memory-layer lookup on one MI355X.

Headline (``value``): lookup tokens/s on the text-study layer, 8,192 tokens,
262,144 fp16 slots (H=4, d_key=256, k=16, d_value=256).  One step is the full
lookup of memory.py:132-193 on inputs already resident in HBM: sub-key
normalisation + packing, scoring (with the query normalisation fused in)
with the two-stage top-k and softmax, and the fp16 gather-weighted-sum.

Also reported in the same JSON line:
  * ``roofline``: the dominant kernel's algorithmic throughput against
    MI355X's published peak, timed with HIP events on its own stream;
  * ``pool_67M``: the large-pool decode lookup (67,108,864 fp16 slots, 34 GB
    in HBM) at 1, 16, 256 and 4,096 tokens, with the gather's HBM roofline;
  * ``cpu_baseline``: the numpy oracle on the host cores over a bounded sample
    of the same workload.

  * ``training_262k``: the training step of the same layer (forward +
    backward + sparse row-wise Adagrad) and the sparse row update alone on
    Zipf(1.1)-skewed routing;
  * ``fact_task_16k_fp32``: the fact-task layer (16,384 fp32 slots, 1,024
    tokens) on fp32 MFMA scoring: the forward read, and a training step whose
    balance and key-diversity terms run on fp32 MFMA tiles;
  * ``key_diversity_67M``: key_diversity_loss and its gradient on the
    67M-slot layer's codebooks (H=4, n=8,192): the n x n Gram tiles on MFMA;
  * ``generation_268M``: end-to-end batched greedy generation, 4-layer
    backbone (d_model 256, 4 heads, FFN x4, vocab 16,384) with memory layers
    1 and 3 reading one 268,435,456-slot fp16 pool (137 GB in HBM), 64
    streams, 128-token prompts, 256 new tokens, every position one
    HIP-graph decode step.

  * ``host_pool_1M``: the host tier (host_pool.py): the text-study lookup
    (8,192 tokens) on a 1,048,576-slot fp16 table in pinned host memory,
    the unique rows copied across the host link by the GPU each step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-large] [--no-train] [--no-generate]
                       [--no-host]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "memory-layer lookups tokens/s at 262k & 67M slots; gather HBM GB/s % peak"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-large", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-train", action="store_true")
    ap.add_argument("--no-generate", action="store_true")
    ap.add_argument("--no-host", action="store_true")
    ap.add_argument("--only", choices=["text_study", "pool_67M_4096", "host_file", "fact_task", "sparse_update",
                                         "cpu_67M", "generation", "train", "stage1", "stage1_67M", "decode"],
                    default=None,
                    help="run one workload alone (for profiler runs) and print its timings")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 512 MiB device copy 10 times (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    return ap.parse_args()


TRAFFIC_FILES = {
    "text_study": os.path.join(ROOT, "profiles", "traffic_text_study_8192.json"),
    "pool_67M_4096": os.path.join(ROOT, "profiles", "traffic_67M_4096.json"),
}


def measured_traffic(kernel, workload="text_study"):
    """HBM bytes per launch of `kernel` on a workload, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE runs recorded in profiles/ (already scaled by the
    copy-kernel calibration); None when not recorded."""
    try:
        with open(TRAFFIC_FILES[workload]) as f:
            rec = json.load(f)
    except (OSError, ValueError, KeyError):
        return None
    k = rec.get("kernels", {}).get(kernel)
    return None if k is None else k.get("hbm_bytes_per_launch")


def copy_calibration(torch):
    n = 512 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": 10}))


_COPY_PEAK = {}


def measured_copy_peak(torch):
    """Bandwidth of a plain 1 GiB device-to-device copy (torch's copy kernel),
    read + written bytes over the time of one copy, best of 3 x 10 launches:
    the measured reference the gather's HBM figure is also reported
    against.  Cached per process."""
    if "GBs" not in _COPY_PEAK:
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
        dst = torch.empty_like(src)
        ms = time_direct(torch, lambda i: dst.copy_(src), 10, 2)
        _COPY_PEAK["GBs"] = 2 * n / (ms * 1e-3) / 1e9
        del src, dst
        torch.cuda.empty_cache()
    return _COPY_PEAK["GBs"]


class Lookup:
    """Preallocated buffers + direct C-ABI calls for one workload.

    ``rotate`` = R independent token batches of M tokens each (queries and
    every output), called in turn: call i works on batch i % R.  Rotating
    batches whose fetched rows total more than the 256 MB Infinity Cache make
    the timed value reads come from HBM rather than from rows a previous call
    left in the cache."""

    def __init__(self, torch, L, *, M, H, n, d_key, d, k, seed, values=None, rotate=1):
        from model_amd import _lib

        self.torch, self.L, self._lib = torch, L, _lib
        self.M, self.H, self.n, self.half, self.d, self.k = M, H, n, d_key // 2, d, k
        self.R = R = max(1, int(rotate))
        dev = "cuda"
        g = torch.Generator(device=dev).manual_seed(seed)
        # hidden ~ N(0,1) [M, 256] through a Xavier-uniform 256 -> H*d_key query projection
        d_model = 256
        hidden = torch.randn((R * M, d_model), generator=g, device=dev)
        lim = math.sqrt(6.0 / (d_model + H * d_key))
        w_q = (torch.rand((d_model, H * d_key), generator=g, device=dev) * 2 - 1) * lim
        self.q = (hidden @ w_q).reshape(R * M, H, 2, self.half).contiguous()
        self.sub_keys = torch.randn((H, 2, n, self.half), generator=g, device=dev) * (self.half ** -0.5)
        if values is None:
            values = torch.empty((n * n, d), dtype=torch.float16, device=dev)
            values.normal_(0.0, 0.02, generator=g)
        self.values = values
        self.T = torch.full((1,), 10.0, device=dev)  # the clamped temperature, a device scalar
        f32, i32, u8 = torch.float32, torch.int32, torch.uint8
        self.packed = torch.empty(L.mpl_packed_keys_bytes(H, n, self.half, _lib.MPL_F16), dtype=u8, device=dev)
        self.ws_bytes = L.mpl_score_select_workspace_bytes(M, H, n, self.half, k)
        self.ws = torch.empty(max(1, self.ws_bytes), dtype=u8, device=dev)
        self.topk_ws_bytes = L.mpl_score_topk_workspace_bytes(M, H, n, self.half, k)
        self.topk_ws = torch.empty(max(1, self.topk_ws_bytes), dtype=u8, device=dev)
        self.sub_idx = torch.empty((R * M, H, 2, k), dtype=i32, device=dev)
        self.sub_scores = torch.empty((R * M, H, 2, k), dtype=f32, device=dev)
        self.flat_idx = torch.empty((R * M, H, k), dtype=i32, device=dev)
        self.slots = torch.empty((R * M, H, k), dtype=i32, device=dev)
        self.weights = torch.empty((R * M, H, k), dtype=f32, device=dev)
        self.out = torch.empty((R * M, d), dtype=f32, device=dev)

    @property
    def stream(self):
        # queried per call: under graph capture the current stream is the capture stream
        return self.torch.cuda.current_stream().cuda_stream

    def _p(self, t, i):
        """Device address of batch i % R of a [R*M, ...] buffer."""
        b = i % self.R
        return t.data_ptr() + b * (t.numel() // self.R) * t.element_size()

    def pack(self, i=0):
        p = self._lib.ptr
        # inference needs only the packed operand, not the fp32 normalised keys
        self._lib.check(self.L.mpl_pack_keys(p(self.sub_keys), self.H, self.n, self.half, self._lib.MPL_F16,
                                             None, p(self.packed), self.stream), "pack")

    def select(self, i=0):
        # raw queries: the scoring kernel l2-normalises them (memory.py:136)
        b, p = self._p, self._lib.ptr
        self._lib.check(self.L.mpl_score_select(
            b(self.q, i), self._lib.MPL_Q_RAW, None, p(self.packed), self.M, self.H, self.n, self.half, self.k,
            self._lib.MPL_F16,
            p(self.T), None, None, p(self.ws), self.ws_bytes, b(self.sub_idx, i), b(self.sub_scores, i),
            b(self.flat_idx, i), b(self.slots, i), b(self.weights, i), self.stream), "select")

    def topk(self, i=0):
        # stage 1 alone (score_topk_kernel, plus split merges when the keys are split)
        b, p = self._p, self._lib.ptr
        self._lib.check(self.L.mpl_score_topk(
            b(self.q, i), self._lib.MPL_Q_RAW, None, p(self.packed), self.M, self.H, self.n, self.half, self.k,
            self._lib.MPL_F16, p(self.T), None, None, p(self.topk_ws), self.topk_ws_bytes, b(self.sub_idx, i),
            b(self.sub_scores, i), self.stream), "topk")

    def gather(self, i=0):
        b = self._p
        self._lib.check(self.L.mpl_gather_wsum(self.values.data_ptr(), self._lib.MPL_F16, self.n * self.n, self.d,
                                               b(self.slots, i), b(self.weights, i), self.M, self.H * self.k, 0,
                                               b(self.out, i), self.stream), "gather")

    def lookup(self, i=0):
        # selection and value read in one call: at H = 4, k = 16 the pair
        # stage and the weighted row sum run as one kernel
        b, p = self._p, self._lib.ptr
        self._lib.check(self.L.mpl_lookup(
            b(self.q, i), self._lib.MPL_Q_RAW, None, p(self.packed), self.M, self.H, self.n, self.half, self.k,
            self._lib.MPL_F16, p(self.T), None, None, p(self.ws), self.ws_bytes, b(self.sub_idx, i),
            b(self.sub_scores, i), b(self.flat_idx, i), b(self.slots, i), b(self.weights, i),
            self.values.data_ptr(), self._lib.MPL_F16, self.d, 0, b(self.out, i), self.stream), "lookup")

    def step(self, i=0):
        self.pack(i)
        self.lookup(i)

    def fill_slots(self):
        """Every batch's slots and weights (for timing the read alone), from
        freshly packed keys."""
        self.pack()
        for i in range(self.R):
            self.select(i)


# Token batches the headline cycles through: 4 x 8,192 tokens of queries
# (134 MB) so that no step reads the queries the step before it read.
HEADLINE_ROTATE = 4


def large_rotation(M):
    """Batches a 67M-slot workload cycles through: enough that the rows one
    replay reads total about 1 GB (4x the 256 MB Infinity Cache), at most 64."""
    per_call = M * 4 * 16 * 256 * 2
    return int(max(1, min(64, math.ceil((1 << 30) / per_call))))


def time_loop(torch, fn, iters, warmup):
    """Average ms per call of fn(i): `iters` calls (i = 0 .. iters-1, so a
    rotating workload cycles through its batches) captured in one HIP graph
    and replayed between HIP events on the current stream (the stream every
    entry point is launched on), so host launch overhead is not measured."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(max(1, warmup)):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(iters):
            fn(i)
    graph.replay()  # warm replay
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    graph.replay()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / iters
    del graph
    return ms


def time_direct(torch, fn, iters, warmup):
    """Average ms per call of fn(i) launched back to back on the current
    stream (no graph), between HIP events on that stream: per call, the
    kernel's duration plus the launch gap between dispatches.  Used for a
    single kernel's roofline; the host enqueues faster than these kernels
    run, so the queue never drains."""
    for i in range(max(1, warmup)):
        fn(i)
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    best = None
    for _ in range(3):
        a.record()
        for i in range(iters):
            fn(i)
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / iters
        best = ms if best is None else min(best, ms)
    return best


def kernel_breakdown(torch, lk, iters):
    lk.fill_slots()
    return {
        "pack_keys_ms": time_loop(torch, lk.pack, iters, 3),
        "score_select_ms": time_loop(torch, lk.select, iters, 3),
        "score_topk_ms": time_loop(torch, lk.topk, iters, 3),
        "gather_wsum_ms": time_loop(torch, lk.gather, iters, 3),
        "lookup_ms": time_loop(torch, lk.lookup, iters, 3),
    }


RIDGE = MFMA_F16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)  # FLOP per byte where the two roofs meet


def topk_algorithmic(lk):
    """Algorithmic work of one stage-1 launch (score_topk_kernel) on M tokens:
    2*H*2*n*half FLOP of scoring per token (2048*n at d_key = 256) and the
    bytes it must move: the fp32 queries read, the fp16 packed sub-keys read
    once, the k (score, id) pairs per codebook written."""
    flops = 2.0 * lk.H * 2 * lk.n * lk.half * lk.M
    nbytes = lk.M * lk.H * 2 * lk.half * 4 + lk.H * 2 * lk.n * lk.half * 2 + lk.M * lk.H * 2 * lk.k * 8
    return flops, nbytes


def roofline_for(lk, br, workload="text_study"):
    """The roofline of the stage-1 scoring kernel (score_topk_kernel), timed
    alone through mpl_score_topk: at the text-study shape the keys are not
    split, so that call is exactly one launch of the kernel.  Its bound is
    set by its arithmetic intensity against the MI355X ridge (312 FLOP/B):
    at n = 512 it is about 200 FLOP/B, so HBM; at n = 8,192 with 4,096 tokens
    it is far above the ridge, so MFMA."""
    flops, nbytes = topk_algorithmic(lk)
    sec = br["score_topk_ms"] * 1e-3
    if flops / nbytes >= RIDGE:
        a = flops / sec / 1e12
        return {"kernel": "score_topk", "bound": "mfma", "achieved": a, "peak": MFMA_F16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": a / MFMA_F16_PEAK_TFLOPS, "traffic": measured_traffic("score_topk", workload),
                "algorithmic_flops": flops, "algorithmic_bytes": nbytes, "flop_per_byte": flops / nbytes}
    a = nbytes / sec / 1e9
    return {"kernel": "score_topk", "bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": a / HBM_PEAK_GBS, "traffic": measured_traffic("score_topk", workload), "algorithmic_bytes": nbytes,
            "algorithmic_flops": flops, "flop_per_byte": flops / nbytes,
            "mfma_frac": flops / sec / 1e12 / MFMA_F16_PEAK_TFLOPS}


def read_algorithmic(lk):
    """Algorithmic bytes of one pair_read_k16 launch (stage 2 fused with the
    value read) on M tokens: the fetched fp16 rows (H*k*d*2 per token), the
    stage-1 lists read (2H*k (score, id) pairs, 8 B each), the slots,
    flat indices and weights written (H*k * 12 B) and the fp32 output row."""
    rows = lk.M * lk.H * lk.k * lk.d * 2
    return rows + lk.M * 2 * lk.H * lk.k * 8 + lk.M * lk.H * lk.k * 12 + lk.M * lk.d * 4, rows


# Random 512-byte rows of a cache-resident 128 MiB table, read by a probe kernel
# with nothing else in it: 37.7 us per 256 MiB (the text-study value read's
# ceiling while its 134 MB table sits in the 256 MB Infinity Cache).
CACHE_RANDOM_ROW_CEILING_GBS = 7100.0


def read_roofline(lk, br, workload="text_study"):
    """Roofline of the fused stage-2 + value-read kernel (pair_read_k16), the
    part of mpl_lookup after stage 1: its time is lookup_ms - score_topk_ms
    (at the text-study shape the keys are not split, so mpl_lookup is one
    score_topk_kernel launch and one pair_read_k16 launch).  HBM-bound by
    its bytes; at this shape the 134 MB table is served by the Infinity
    Cache, so the measured random-row ceiling of that cache is given beside
    the HBM peak."""
    nbytes, rows = read_algorithmic(lk)
    ms = br["lookup_ms"] - br["score_topk_ms"]
    a = nbytes / (ms * 1e-3) / 1e9
    return {"kernel": "pair_read_k16", "bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": a / HBM_PEAK_GBS, "traffic": measured_traffic("pair_read_k16", workload),
            "algorithmic_bytes": nbytes, "row_bytes": rows, "ms_per_launch": ms,
            "timing": "lookup_ms - score_topk_ms (HIP events over graph-replayed launches)",
            "served_from": "Infinity Cache (the 134 MB table stays resident between steps)",
            "cache_random_row_ceiling_GBs": CACHE_RANDOM_ROW_CEILING_GBS,
            "frac_of_cache_ceiling": a / CACHE_RANDOM_ROW_CEILING_GBS}


def dominant_roofline(lk, br):
    """The roofline object of the kernel that takes the larger share of the
    text-study step: stage 1 (score_topk_kernel) or the fused stage 2 + read
    (pair_read_k16); the other is returned beside it."""
    r1 = roofline_for(lk, br)
    r2 = read_roofline(lk, br)
    t1, t2 = br["score_topk_ms"], r2["ms_per_launch"]
    r1["ms_per_launch"] = t1
    return (r1, r2) if t1 >= t2 else (r2, r1)


def gather_roofline(torch, lk, br, iters):
    """HBM roofline of the value read alone (gather_wsum_kernel, one launch of
    mpl_gather_wsum) over rotating batches: algorithmic bytes = the fetched
    rows, M * H * k * d * 2 B.  ``achieved`` is from back-to-back launches
    (the kernel duration plus the dispatch gap); the graph-replayed figure of
    the kernel breakdown, which adds a graph node's gap, is given beside it,
    and so is the fraction of a measured device-copy bandwidth."""
    gb = lk.M * lk.H * lk.k * lk.d * 2
    ms = time_direct(torch, lk.gather, iters, lk.R)
    a = gb / (ms * 1e-3) / 1e9
    cp = measured_copy_peak(torch)
    return {"kernel": "gather_wsum", "bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": a / HBM_PEAK_GBS, "copy_peak_GBs": cp, "frac_of_copy_peak": a / cp,
            "ms_per_launch": ms, "algorithmic_bytes": gb,
            "traffic": measured_traffic("gather_wsum", "pool_67M_4096") if (lk.n, lk.M) == (8192, 4096) else None,
            "graph_replay_GBs": gb / (br["gather_wsum_ms"] * 1e-3) / 1e9, "rotating_batches": lk.R,
            "distinct_row_bytes_per_replay": gb * lk.R}


def zipf_slots(M, H, k, N, s=1.1, seed=5):
    """[M, H, k] slots drawn by rank with p(r) ~ r^-s over 1..N through a fixed
    random permutation, distinct within each (token, head)."""
    rng = np.random.default_rng(seed)
    cdf = np.cumsum(np.arange(1, N + 1, dtype=np.float64) ** -s)
    cdf /= cdf[-1]
    perm = rng.permutation(N)
    G = M * H
    draws = np.minimum(np.searchsorted(cdf, rng.random((G, 8 * k))), N - 1)
    order = np.argsort(draws, axis=1, kind="stable")
    sd = np.take_along_axis(draws, order, 1)
    dup_s = np.zeros_like(sd, dtype=bool)
    dup_s[:, 1:] = sd[:, 1:] == sd[:, :-1]
    dup = np.empty_like(dup_s)
    np.put_along_axis(dup, order, dup_s, 1)
    nd = ~dup
    c = np.cumsum(nd, axis=1)
    out = np.empty((G, k), dtype=np.int64)
    full = c[:, -1] >= k
    out[full] = draws[full][(nd & (c <= k))[full]].reshape(-1, k)
    for g in np.flatnonzero(~full):
        first = draws[g][nd[g]]
        out[g] = np.concatenate([first, np.setdiff1d(np.arange(N), first)[: k - first.shape[0]]])
    return perm[out].reshape(M, H, k).astype(np.int32)


def sparse_update_bench(torch, iters):
    """The sparse value update of the training config on Zipf(1.1) routing:
    merge of 524,288 fetches (8,192 tokens x 4 heads x 16) into rows of a
    262,144-slot table, global-norm clip, row-wise Adagrad on an fp32 master
    with the fp16 table refreshed."""
    from model_amd import rows as R

    M, H, k, N, d = 8192, 4, 16, 262144, 256
    dev = "cuda"
    slots = torch.as_tensor(zipf_slots(M, H, k, N), device=dev)
    g = torch.Generator(device=dev).manual_seed(4)
    w = torch.rand((M, H, k), generator=g, device=dev)
    w = w / w.sum(-1, keepdim=True)
    g_out = torch.randn((M, d), generator=g, device=dev) * 1e-3
    values = torch.empty((N, d), dtype=torch.float16, device=dev).normal_(0.0, 0.02, generator=g)
    master = values.float()
    acc = torch.zeros(N, device=dev)
    rest = torch.tensor([1e-4], device=dev)

    # as SparseRowUpdate runs it: the padding rows [U, cap) are left
    # unwritten, since the optimizers never read them
    def step(i=0):
        m = R.merge_fetches(slots, w, g_out, N, zero_padding=False)
        sg = R.clip_scale(m.row_sq, rest, 1.0)
        R.rowwise_adagrad(values, acc, m.uniq, m.rows, 3e-3, master=master, grad_scale=sg[0:1])
        return m

    m = step()
    torch.cuda.synchronize()
    U = int(m.num_unique.cpu()[0])
    ms = time_loop(torch, step, iters, 3)
    P = M * H * k
    alg = P * 8 + M * d * 4 + U * (2 * d * 4 + d * 2 + 8)

    # the same merge and clip followed by the lazy Adam step (train.py:417-426)
    m1 = torch.zeros((N, d), device=dev)
    m2 = torch.zeros((N, d), device=dev)

    def step_adam(i=0):
        mm = R.merge_fetches(slots, w, g_out, N, zero_padding=False)
        sg = R.clip_scale(mm.row_sq, rest, 1.0)
        R.lazy_adam(values, m1, m2, mm.uniq, mm.rows, 3e-3, 7, master=master, grad_scale=sg[0:1])

    ms_adam = time_loop(torch, step_adam, iters, 3)
    # per row: the merged row read, master and both moments read and written, fp16 row written
    alg_adam = P * 8 + M * d * 4 + U * (7 * d * 4 + d * 2)
    return {"workload": "sparse row update: 524,288 Zipf(1.1) fetches (8,192 tokens x 4 heads x 16), "
                        "262,144-slot fp16 table + fp32 master, d=256, row-wise Adagrad",
            "unique_rows": U, "ms": ms, "fetches_per_s": P / (ms * 1e-3),
            "hbm": {"algorithmic_bytes": alg, "achieved_GBs": alg / (ms * 1e-3) / 1e9,
                    "frac": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
            # the merge reads one fp32 g_out row (d * 4 B) per fetch; the 8 MB g_out is
            # cache-resident, so these bytes come from L2 and the Infinity Cache, not HBM
            "cache_bytes": {"g_out_rows_per_fetch": P * d * 4,
                            "achieved_GBs": (alg + P * d * 4) / (ms * 1e-3) / 1e9,
                            "note": "algorithmic HBM bytes plus the per-fetch g_out row reads"},
            "lazy_adam": {"ms": ms_adam, "fetches_per_s": P / (ms_adam * 1e-3),
                          "hbm": {"algorithmic_bytes": alg_adam, "achieved_GBs": alg_adam / (ms_adam * 1e-3) / 1e9,
                                  "frac": alg_adam / (ms_adam * 1e-3) / 1e9 / HBM_PEAK_GBS}}}


def train_step_bench(torch, iters):
    """Forward + backward of the text-study layer in training (8,192 tokens,
    262,144 fp16 slots, H=4, d_key=256, k=16, routing noise on as in the
    reference's training step (train=True, routing_noise 1.0), balance
    coefficient 0.01, sparse value gradient through a probe) followed by the
    sparse row update (merge, clip, row-wise Adagrad on the fp32 master)."""
    from model_amd import rows as R
    from model_amd.memory import MemoryPool, key_diversity_loss

    M, H, n, d_key, d, k = 8192, 4, 512, 256, 256, 16
    dev = "cuda"
    pool = MemoryPool(n, H, d_key, d, k, values_dtype=torch.float16)
    g = torch.Generator(device=dev).manual_seed(0)
    keys = (torch.randn((H, 2, n, d_key // 2), generator=g, device=dev) * (d_key // 2) ** -0.5).requires_grad_(True)
    values = torch.empty((n * n, d), dtype=torch.float16, device=dev).normal_(0.0, 0.02, generator=g)
    log_t = torch.tensor(math.log(10.0), device=dev, requires_grad=True)
    params = {"sub_keys": keys, "values": values, "log_temperature": log_t}
    hidden = torch.randn((M, 256), generator=g, device=dev)
    lim = math.sqrt(6.0 / (256 + H * d_key))
    w_q = ((torch.rand((256, H * d_key), generator=g, device=dev) * 2 - 1) * lim).requires_grad_(True)
    g_out = torch.randn((M, d), generator=g, device=dev) * 1e-3
    upd = R.SparseRowUpdate(values, lr=1e-3, pool_lr_mult=3.0, warmup_steps=0, steps=1000, grad_clip=1.0)

    def step():
        q = (hidden @ w_q).reshape(M, H, d_key)
        probe = torch.zeros((M, d), device=dev, requires_grad=True)
        out, aux = pool.apply({"params": params}, q, train=True, sparse_grad=True)
        loss = ((out + probe) * g_out).sum() + 0.01 * aux["balance_loss"] + 0.01 * key_diversity_loss(keys)
        gw, gk, gt, gp = torch.autograd.grad(loss, [w_q, keys, log_t, probe])
        rest = R.sum_squares([gw, gk, gt])
        # the per-step slot counts (memory.py:215) come from the merge's sort
        upd({"slots": [aux["slots"]], "weights": [aux["weights"]]}, {0: gp}, [0], rest_sq=rest, count_slots=True)

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        step()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / iters

    # The same step without torch autograd (MemoryPool.forward_backward with
    # the key diversity term; the projection's gradient as a product),
    # captured in one HIP graph and replayed.
    g_bal = torch.full((), 0.01, device=dev)
    g_div = torch.full((), 0.01, device=dev)
    side = torch.cuda.Stream()  # default priorities
    side2 = torch.cuda.Stream()

    def step_graph(_i):
        with torch.no_grad():
            cur = torch.cuda.current_stream()
            q = (hidden @ w_q).reshape(M, H, d_key)
            pending = {}

            def start_merge(aux):  # the sparse row merge beside the dense backward
                side.wait_stream(cur)
                with torch.cuda.stream(side):
                    pending["m"] = upd.merge({"slots": [aux["slots"]], "weights": [aux["weights"]]}, {0: g_out}, [0],
                                             count_slots=True)

            def start_wgrad(dq):  # the projection's weight gradient beside the sub-key passes
                side2.wait_stream(cur)
                dq.record_stream(side2)
                with torch.cuda.stream(side2):
                    pending["gw"] = hidden.t() @ dq.reshape(M, H * d_key)

            # the key diversity term's gradient joins d sub_keys inside the call
            out, aux, (dq, gk, dlt) = pool.forward_backward({"params": params}, q, g_out, g_bal, train=True,
                                                            g_diversity=g_div, on_forward=start_merge,
                                                            on_dq=start_wgrad)
            cur.wait_stream(side)
            cur.wait_stream(side2)
            gw = pending["gw"]
            gw.record_stream(cur)
            # the dense gradients' norm in the clip's own pass (no memset node)
            upd.apply(pending["m"], dense_grads=[gw, gk, dlt])

    ms_graph = time_loop(torch, step_graph, iters, 3)
    return {"workload": "training step of the text-study layer: 8,192 tokens, 262,144 fp16 slots + fp32 master, "
                        "forward with Gumbel routing noise + backward (queries through a 256->1024 projection, "
                        "sub-keys, log-temperature, "
                        "balance loss 0.01, key diversity loss 0.01, probe gradient) + sparse row-wise Adagrad "
                        "+ routing statistics (sub-key counts, per-slot fetch counts from the row merge)",
            "ms_per_step": ms, "tokens_per_s": M / (ms * 1e-3), "timing": "eager, HIP events",
            "graph_ms_per_step": ms_graph, "graph_tokens_per_s": M / (ms_graph * 1e-3),
            "graph_timing": "the same step through MemoryPool.forward_backward (no torch autograd; the sparse row "
                            "merge and the projection's weight gradient on two more streams beside the dense "
                            "backward), "
                            f"{iters} steps captured in one HIP graph and replayed between HIP events"}


def fact_task_bench(torch, iters):
    """The fact-task layer on the GPU, fp32 throughout (fp32 table, fp32
    MFMA scoring): 1,024 tokens (B=8, T=128), 16,384 slots (n_sub_keys=128),
    H=4, d_key=256, k=16, d_value=256.  `lookup`: the forward read alone.
    `train_step`: forward with routing noise + backward through a 256->1024
    query projection, the sub-keys and log-temperature, with the balance loss
    (0.01) and the fp32 key-diversity loss (0.01), whose dense terms run on
    v_mfma_f32_32x32x2_f32 tiles."""
    from model_amd.memory import MemoryPool, key_diversity_loss

    M, H, n, d_key, d, k = 1024, 4, 128, 256, 256, 16
    dev = "cuda"
    pool = MemoryPool(n, H, d_key, d, k, values_dtype=torch.float32)
    assert pool.score_dtype == torch.float32
    g = torch.Generator(device=dev).manual_seed(11)
    keys = (torch.randn((H, 2, n, d_key // 2), generator=g, device=dev) * (d_key // 2) ** -0.5).requires_grad_(True)
    values = torch.empty((n * n, d), dtype=torch.float32, device=dev).normal_(0.0, 0.02, generator=g)
    log_t = torch.tensor(math.log(10.0), device=dev, requires_grad=True)
    params = {"sub_keys": keys, "values": values, "log_temperature": log_t}
    hidden = torch.randn((M, 256), generator=g, device=dev)
    lim = math.sqrt(6.0 / (256 + H * d_key))
    w_q = ((torch.rand((256, H * d_key), generator=g, device=dev) * 2 - 1) * lim).requires_grad_(True)
    g_out = torch.randn((M, d), generator=g, device=dev) * 1e-3
    q0 = (hidden @ w_q).detach().reshape(M, H, d_key).contiguous()

    def fwd(i=0):
        pool.lookup(params, q0)

    def step(i=0):
        q = (hidden @ w_q).reshape(M, H, d_key)
        out, aux = pool.apply({"params": params}, q, train=True, rngs={"routing": i})
        loss = (out * g_out).sum() + 0.01 * aux["balance_loss"] + 0.01 * key_diversity_loss(keys, torch.float32)
        torch.autograd.grad(loss, [w_q, keys, log_t])

    def eager(fn, n_iter):  # no graph capture: timed as it runs, median of 5 runs of n_iter calls
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        runs = []
        for _ in range(5):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            for i in range(n_iter):
                fn(i)
            b.record()
            torch.cuda.synchronize()
            runs.append(a.elapsed_time(b) / n_iter)
        return sorted(runs)[2]

    ms_fwd = eager(fwd, iters * 4)
    ms_step = eager(step, iters)
    return {"workload": "fact-task layer, fp32: 1,024 tokens, 16,384 fp32 slots, H=4, d_key=256, k=16, d_value=256",
            "lookup": {"ms": ms_fwd, "tokens_per_s": M / (ms_fwd * 1e-3)},
            "train_step": {"ms": ms_step, "tokens_per_s": M / (ms_step * 1e-3),
                           "what": "forward with routing noise + backward, balance 0.01 and fp32 key diversity "
                                   "0.01 on fp32 MFMA tiles (no value update)"},
            "timing": "eager, HIP events, median of 5 runs"}


def key_diversity_bench(torch, iters):
    """key_diversity_loss and its gradient with respect to the normalised
    sub-keys (memory.py:230-240) for the 67M-slot layer's codebooks (H=4,
    n=8,192, d_key=256): per codebook the Gram tiles K K^T and the product
    (G - diag G) K, each 2 n^2 (d_key/2) FLOP, on fp16 MFMA."""
    from model_amd import _lib
    from model_amd._lib import check, ptr

    L = _lib.lib()
    H, n, half = 4, 8192, 128
    g = torch.Generator(device="cuda").manual_seed(5)
    keys = torch.randn((H, 2, n, half), generator=g, device="cuda")
    k_hat = torch.empty_like(keys)
    packed = torch.empty(L.mpl_packed_keys_bytes(H, n, half, _lib.MPL_F16), dtype=torch.uint8, device="cuda")
    check(L.mpl_pack_keys(ptr(keys), H, n, half, _lib.MPL_F16, ptr(k_hat), ptr(packed),
                          _lib.stream_ptr(keys.device)), "mpl_pack_keys")
    wsb = L.mpl_key_diversity_workspace_bytes(H, n, half, _lib.MPL_F16)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    loss = torch.empty(1, dtype=torch.float32, device="cuda")
    dk = torch.empty_like(keys)

    def fn(i=0):
        check(L.mpl_key_diversity(ptr(k_hat), ptr(packed), H, n, half, _lib.MPL_F16, ptr(ws), wsb, ptr(loss),
                                  ptr(dk), _lib.stream_ptr(keys.device)), "mpl_key_diversity")

    ms = time_loop(torch, fn, iters, 3)
    flops = 2 * (2.0 * 2 * H * n * n * half)
    tf = flops / (ms * 1e-3) / 1e12
    return {"workload": "key_diversity_loss + d/d k_hat, H=4, n=8,192, d_key=256 (2 x 137.4 GFLOP)",
            "ms": ms, "achieved_tflops": tf, "peak_tflops": MFMA_F16_PEAK_TFLOPS, "frac": tf / MFMA_F16_PEAK_TFLOPS}


def host_pool_bench(torch, iters):
    """The lookup with the value table in pinned host memory (host_pool.py,
    RAM mode): select on the GPU, then the unique rows cross the host link
    once (mpl_unique_slots + mpl_gather_rows reading the pinned table) and
    the weighted sum runs on the staged rows."""
    from model_amd import _lib
    from model_amd import host_pool as hp

    L = _lib.lib()
    M, H, n, d_key, d, k = 8192, 4, 1024, 256, 256, 16
    N = n * n
    pool = hp.HostPool(N, d, dtype=np.float16, seed=0, optimizer="rowwise_adagrad")
    lk = Lookup(torch, L, M=M, H=H, n=n, d_key=d_key, d=d, k=k, seed=0,
                values=torch.empty((16, d), dtype=torch.float16, device="cuda"))
    lk.pack()
    lk.select()
    staged = {}

    def stage(i=0):
        staged["rows"], staged["inv"], staged["num"] = pool.stage(lk.slots)

    def read(i=0):
        _lib.check(L.mpl_gather_wsum(_lib.ptr(staged["rows"]), _lib.MPL_F16, staged["rows"].shape[0], d,
                                     _lib.ptr(staged["inv"]), _lib.ptr(lk.weights), M, H * k, 0, _lib.ptr(lk.out),
                                     lk.stream), "gather")

    def step(i=0):
        lk.pack()
        lk.select()
        stage()
        read()

    stage()
    torch.cuda.synchronize()
    U = int(staged["num"].item())
    t_stage = time_loop(torch, stage, iters, 2)
    t_step = time_loop(torch, step, iters, 2)
    link = U * d * 2 / (t_stage * 1e-3) / 1e9
    # the host tier's training step: row-wise Adagrad of the U touched rows,
    # in place on the pinned table (train.py:250-258 -> host_pool.py:143-152)
    flat = lk.slots.reshape(-1)
    uniq = torch.unique(flat).to(torch.int32)
    grads = torch.randn((uniq.numel(), d), device="cuda") * 1e-3
    t_upd = time_loop(torch, lambda i=0: pool.update(uniq, grads, 1, 1e-3), iters, 2)
    upd_bytes = uniq.numel() * (2 * d * 2 + 2 * 4)  # fp16 row read + write, acc read + write, across the link
    del pool
    return {"workload": "text-study lookup (8,192 tokens, H=4, k=16) on a 1,048,576-slot fp16 table in pinned "
                        "host memory (RAM mode of the host tier), and the row-wise Adagrad step of the touched rows",
            "unique_rows": U, "stage_ms": t_stage, "host_link_GBs": link, "ms_per_step": t_step,
            "tokens_per_s": M / (t_step * 1e-3),
            "update_ms": t_upd, "update_rows_per_s": uniq.numel() / (t_upd * 1e-3),
            "update_link_GBs": upd_bytes / (t_upd * 1e-3) / 1e9}


def host_pool_file_bench(torch, iters):
    """The host tier's file mode (the reference's pool directory of .npy
    files): the text-study lookup's unique rows read from a 1,048,576-slot
    fp16 values.npy by the library's row-file reader into pinned staging and
    copied to the GPU, with the page cache warm and after evicting it, and
    the row-wise Adagrad step of those rows (read, GPU step on the staged
    rows, write back)."""
    import shutil
    import tempfile

    from model_amd import _lib
    from model_amd import host_pool as hp

    L = _lib.lib()
    M, H, n, d_key, d, k = 8192, 4, 1024, 256, 256, 16
    N = n * n
    tmp = tempfile.mkdtemp(prefix="mpl_pool_", dir=os.environ.get("TMPDIR", "/tmp"))
    try:
        pool = hp.HostPool(N, d, path=tmp, dtype=np.float16, seed=0, optimizer="rowwise_adagrad")
        lk = Lookup(torch, L, M=M, H=H, n=n, d_key=d_key, d=d, k=k, seed=0,
                    values=torch.empty((16, d), dtype=torch.float16, device="cuda"))
        lk.pack()
        lk.select()
        _, _, num = pool.stage(lk.slots)
        torch.cuda.synchronize()
        U = int(num.item())

        def timed(fn, reps, before=None):
            best = None
            for _ in range(reps):
                if before is not None:
                    before()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                dt = time.perf_counter() - t0
                best = dt if best is None else min(best, dt)
            return best * 1e3

        warm = timed(lambda: pool.stage(lk.slots), iters)
        cold = timed(lambda: pool.stage(lk.slots), 3, before=pool.evict_page_cache)
        # the same reads with O_DIRECT (no page cache: every row from the
        # drive), for the whole batch and for a decode-sized one (64 tokens)
        direct = {}
        ddir = hp.HostPool(N, d, path=tmp, dtype=np.float16, trainable=False, direct_io=True,
                           name="bench-direct") if pool._arrays["values"].direct_supported else None
        dec = lk.slots[:64]
        _, _, num_dec = pool.stage(dec)
        torch.cuda.synchronize()
        U_dec = int(num_dec.item())
        direct["decode_unique_rows"] = U_dec
        direct["decode_stage_warm_ms"] = timed(lambda: pool.stage(dec), iters)
        if ddir is not None:
            direct["stage_direct_ms"] = timed(lambda: ddir.stage(lk.slots), 3)
            direct["stage_direct_row_GBs"] = U * d * 2 / (direct["stage_direct_ms"] * 1e-3) / 1e9
            direct["decode_stage_direct_ms"] = timed(lambda: ddir.stage(dec), iters)
            ddir.close()
        uniq = torch.unique(lk.slots.reshape(-1)).to(torch.int32)
        grads = torch.randn((uniq.numel(), d), device="cuda") * 1e-3
        upd = timed(lambda: pool.update(uniq, grads, 1, 1e-3), max(3, iters // 2))
        pool.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    row_bytes = d * 2
    return {"workload": "text-study lookup (8,192 tokens, H=4, k=16) reading a 1,048,576-slot fp16 values.npy "
                        "(file mode of the host tier), and the row-wise Adagrad step of the touched rows",
            "unique_rows": U, "stage_warm_ms": warm, "stage_warm_GBs": U * row_bytes / (warm * 1e-3) / 1e9,
            "stage_after_evict_ms": cold, "stage_after_evict_GBs": U * row_bytes / (cold * 1e-3) / 1e9,
            "update_ms": upd, "update_rows_per_s": uniq.numel() / (upd * 1e-3),
            "note": "evict_page_cache is advisory (posix_fadvise DONTNEED); where the file system keeps the "
                    "pages (e.g. tmpfs) the 'after evict' read is a page-cache read too",
            "direct_io": direct if ddir is not None else dict(direct, unsupported="O_DIRECT refused here"),
            "direct_note": "direct_io reads 4 KiB-aligned spans around the rows with O_DIRECT (no page cache); "
                           "decode_*: the unique rows of the first 64 tokens (4 heads x 16 rows each)",
            "io_threads": hp._IO_THREADS, "direct_io_threads": hp._DIRECT_THREADS, "dir": os.path.dirname(tmp)}


def generation_bench(torch):
    """Batched greedy generation through the backbone mirror
    (model_amd/model.py, generate.py) with two memory layers on a
    268,435,456-slot fp16 pool filled in place with N(0, 0.02)."""
    from model_amd.generate import Generator
    from model_amd.model import MemoryPoolLM, ModelConfig

    n, d, B, P, new = 16384, 256, 64, 128, 256
    cfg = ModelConfig(vocab_size=16384, max_len=P + new, d_model=256, n_layers=4, n_heads=4, ffn_mult=4,
                      memory_layers=(1, 3), n_sub_keys=n, pool_heads=4, d_key=256, d_value=d, top_k=16,
                      values_dtype=torch.float16)
    g = torch.Generator(device="cuda").manual_seed(7)
    values = torch.empty((n * n, d), dtype=torch.float16, device="cuda")
    values.normal_(0.0, 0.02, generator=g)
    params = MemoryPoolLM(cfg).init(0, pool_values=values)
    gen = Generator(cfg, params, batch_size=B)
    prompt = torch.randint(0, cfg.vocab_size, (B, P), generator=g, device="cuda")
    gen.generate(prompt[:, :8], n_new=4, keep_logits=False)  # capture + warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    res = gen.generate(prompt, n_new=new, keep_logits=False)
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    steps = P + new - 1
    out = {"workload": "greedy generation: 4-layer backbone (d_model 256, 4 heads, FFN x4, vocab 16,384), "
                       "memory layers 1 and 3, 268,435,456-slot fp16 pool (137 GB), H=4, k=16, 64 streams, "
                       "128-token prompts, 256 new tokens (383 decode steps, one HIP graph per step)",
           "seconds": sec, "ms_per_step": 1e3 * sec / steps, "generated_tokens_per_s": B * new / sec,
           "processed_tokens_per_s": B * steps / sec, "tokens_shape": list(res["tokens"].shape)}
    del gen, params, values
    torch.cuda.empty_cache()
    return out


def host_info():
    """Host cores and model (os.cpu_count() and lscpu)."""
    info = {"os_cpu_count": os.cpu_count()}
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            if key.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)"):
                info["lscpu_" + key.strip().lower().replace("(s)", "s").replace(" ", "_")] = val.strip()
    except Exception as e:  # pragma: no cover
        info["lscpu_error"] = str(e)
    return info


def cpu_workers():
    """Worker threads for the CPU baselines: every core this process may use
    (OMP_NUM_THREADS caps it where the box shares its cores between GPUs)."""
    n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(cap))) if cap and cap.isdigit() else n


def _cpu_run(task, chunks, seconds, workers):
    """Calls task(i) for i = 0, 1, ... on `workers` threads (numpy releases
    the GIL in its sorts and BLAS calls; BLAS itself is held to one thread
    per worker) until `seconds` have passed; returns (tasks done, seconds)."""
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    done, t0 = 0, time.perf_counter()
    with threadpool_limits(1), ThreadPoolExecutor(workers) as ex:
        while True:
            list(ex.map(task, range(done, done + chunks)))
            done += chunks
            el = time.perf_counter() - t0
            if el >= seconds:
                return done, el


def cpu_lookup_baseline(seconds: float, *, n, values_dtype, label):
    """The numpy oracle (oracle/lookup.py, memory.py:132-193) on the host
    cores: scoring on BLAS, top-k by partition and stable sort, the weighted
    row read, on chunks of 256 tokens, one chunk per worker at a time."""
    from oracle import lookup as ol

    workers = cpu_workers()
    rng = np.random.default_rng(0)
    H, half, k, d, chunk = 4, 128, 16, 256, 256
    keys = (rng.standard_normal((H, 2, n, half)) * half ** -0.5).astype(np.float32)
    values = (rng.standard_normal((n * n, d)) * 0.02).astype(values_dtype)
    w_q = ((rng.random((256, H * 2 * half)) * 2 - 1) * math.sqrt(6.0 / (256 + H * 2 * half))).astype(np.float32)
    qs = [(np.random.default_rng(100 + i).standard_normal((chunk, 256)).astype(np.float32) @ w_q)
          .reshape(chunk, H, 2 * half) for i in range(workers)]

    def task(i):
        ol.lookup_forward(qs[i % workers], keys, values, np.log(10.0), top_k_=k, with_dense=False)

    done, el = _cpu_run(task, workers, seconds, workers)
    return {"value": done * chunk / el, "unit": "tokens/s", "cores": workers, "kind": "port",
            "sample": f"{done} chunks x {chunk} tokens of the {label} layer ({n * n:,} {np.dtype(values_dtype).name} "
                      f"slots, H=4, d_key=256, k=16) through the numpy oracle on {workers} threads "
                      f"(BLAS one thread each), {el:.1f} s",
            "host": host_info()}


def cpu_lookup_67m_baseline(seconds: float):
    """The numpy oracle at the 67M-slot layer (n = 8,192, H = 4, d_key = 256,
    k = 16, fp16 rows of d = 256), 4,096-token batches as on the GPU, timed
    on chunks of 64 tokens, one per worker at a time.  The 34 GB table is
    not materialised on the host: it is the hash-defined table the GPU
    benchmark fills (seed 3, scale 0.02), so before the clock starts the
    rows each chunk selects are regenerated (oracle/hashinit.py) into a
    compact array; the timed work is the whole lookup (scoring on BLAS,
    both top-k stages, softmax) plus the weighted read of those rows."""
    from oracle import hashinit as hi
    from oracle import lookup as ol

    workers = cpu_workers()
    rng = np.random.default_rng(0)
    H, half, k, d, n, chunk = 4, 128, 16, 256, 8192, 64
    keys = (rng.standard_normal((H, 2, n, half)) * half ** -0.5).astype(np.float32)
    w_q = ((rng.random((256, H * 2 * half)) * 2 - 1) * math.sqrt(6.0 / (256 + H * 2 * half))).astype(np.float32)
    qs, tabs = [], []
    for i in range(workers):
        q = (np.random.default_rng(100 + i).standard_normal((chunk, 256)).astype(np.float32) @ w_q)
        q = q.reshape(chunk, H, 2 * half)
        sel = ol.lookup_forward(q, keys, None, np.log(10.0), top_k_=k, with_dense=False)
        uniq, inv = np.unique(sel["slots"], return_inverse=True)
        qs.append(q)
        tabs.append((hi.hash_normal_rows(3, uniq, d, 0.02), inv.reshape(sel["slots"].shape)))

    def task(i):
        rows, inv = tabs[i % workers]
        res = ol.lookup_forward(qs[i % workers], keys, None, np.log(10.0), top_k_=k, with_dense=False)
        ol.gather_wsum(rows, inv, res["weights"])

    done, el = _cpu_run(task, workers, seconds, workers)
    return {"value": done * chunk / el, "unit": "tokens/s", "cores": workers, "kind": "port",
            "sample": f"{done} chunks x {chunk} tokens of the 67M-slot layer (67,108,864 fp16 slots, n=8,192, H=4, "
                      f"d_key=256, k=16) through the numpy oracle on {workers} threads (BLAS one thread each), "
                      f"{el:.1f} s; the selected rows regenerated from the hash table before timing",
            "host": host_info()}


def cpu_train_baseline(seconds: float):
    """The training step of the 262,144-slot layer through the numpy oracle:
    forward with Gumbel routing noise (memory.py:132-193), the balance loss's
    statistics (memory.py:196-213), the backward (oracle/backward.py) on
    chunks of 256 tokens across the cores, then the sparse row merge, clip and
    row-wise Adagrad of the step's fetches (train.py:146-172, 395-416).  One
    step = 2,048 tokens."""
    from oracle import backward as ob
    from oracle import lookup as ol
    from oracle import rows as orows

    workers = cpu_workers()
    rng = np.random.default_rng(0)
    H, n, half, k, d, chunk, per_step = 4, 512, 128, 16, 256, 256, 2048
    N = n * n
    keys = (rng.standard_normal((H, 2, n, half)) * half ** -0.5).astype(np.float32)
    values = (rng.standard_normal((N, d)) * 0.02).astype(np.float16)
    master = values.astype(np.float32)
    acc = np.zeros(N, np.float32)
    q = rng.standard_normal((per_step, H, 2 * half)).astype(np.float32)
    g = (rng.standard_normal((per_step, d)) * 1e-3).astype(np.float32)
    gum = -np.log(-np.log(rng.random((per_step, H, 2, n)).clip(1e-30, 1 - 1e-7))).astype(np.float32)
    parts = per_step // chunk

    def chunk_fb(j):
        sl = slice(j * chunk, (j + 1) * chunk)
        res = ol.lookup_forward(q[sl], keys, values, np.log(10.0), top_k_=k, gumbel=gum[sl], noise_coef=1.0)
        f = ol.aux_stats(res, n=n, noisy=True)["_f"]
        ob.lookup_backward(res, values, g[sl], n=n, g_balance=0.01, f=f, dtype=np.float32)
        return res["slots"], res["weights"]

    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    steps, t0 = 0, time.perf_counter()
    with threadpool_limits(1), ThreadPoolExecutor(workers) as ex:
        while True:
            outs = list(ex.map(chunk_fb, range(parts)))
            slots = np.concatenate([o[0] for o in outs])
            wts = np.concatenate([o[1] for o in outs])
            uniq, rows = orows.fetched_row_grads([slots], [wts], [g], N)
            sg, _ = orows.clip_scale(1e-4, rows, 1.0)
            orows.rowwise_adagrad(values, acc, uniq, rows * np.float32(sg), 3e-3, master=master)
            steps += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
    return {"value": steps * per_step / el, "unit": "tokens/s", "cores": min(workers, parts), "kind": "port",
            "sample": f"{steps} steps x {per_step} tokens of the 262,144-slot training layer (fp16 table, fp32 "
                      f"master): oracle forward with noise + balance statistics + backward on {parts} chunks of "
                      f"{chunk} tokens across {min(workers, parts)} threads, then the row merge, clip and "
                      f"row-wise Adagrad (single thread), {el:.1f} s",
            "host": host_info()}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the lookup shards over tokens; one GPU is what is built and measured).", file=sys.stderr)
        sys.exit(2)
    import torch

    from model_amd import _lib
    from model_amd.hashinit import hash_normal_

    L = _lib.lib()
    torch.cuda.set_device(0)
    if args.copy_calibration:
        copy_calibration(torch)
        return

    if args.only == "text_study":
        lk = Lookup(torch, L, M=8192, H=4, n=512, d_key=256, d=256, k=16, seed=0, rotate=HEADLINE_ROTATE)
        print(json.dumps({"only": args.only, "ms_per_step": time_loop(torch, lk.step, args.steps, args.warmup),
                          "kernels": kernel_breakdown(torch, lk, args.steps)}))
        return
    if args.only in ("stage1", "stage1_67M"):
        # stage 1 alone (mpl_score_topk) for counter runs: the text-study shape
        # (8,192 tokens, n = 512) or the 67M-slot key width at 4,096 tokens
        # (n = 8,192; no value table is needed), 8 launches after warm-up
        if args.only == "stage1":
            lk = Lookup(torch, L, M=8192, H=4, n=512, d_key=256, d=256, k=16, seed=0, rotate=HEADLINE_ROTATE)
        else:
            vals = torch.empty((1, 256), dtype=torch.float16, device="cuda")
            lk = Lookup(torch, L, M=4096, H=4, n=8192, d_key=256, d=256, k=16, seed=4106, values=vals, rotate=4)
        lk.pack()
        for i in range(3):
            lk.topk(i % lk.R)
        torch.cuda.synchronize()
        for i in range(8):
            lk.topk(i % lk.R)
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, "score_topk_ms": time_loop(torch, lk.topk, 20, 3)}))
        return
    if args.only == "train":
        print(json.dumps({"only": args.only, "train_step": train_step_bench(torch, 10)}))
        return
    if args.only == "generation":
        print(json.dumps({"only": args.only, "generation_268M": generation_bench(torch)}))
        return
    if args.only == "cpu_67M":
        print(json.dumps({"only": args.only, "pool_67M_4096": cpu_lookup_67m_baseline(args.cpu_seconds / 2)}))
        return
    if args.only == "sparse_update":
        print(json.dumps({"only": args.only, "sparse_update_zipf": sparse_update_bench(torch, args.steps)}))
        return
    if args.only == "fact_task":
        print(json.dumps({"only": args.only, "fact_task_16k_fp32": fact_task_bench(torch, 10)}))
        return
    if args.only == "host_file":
        print(json.dumps({"only": args.only, "host_pool_file_1M": host_pool_file_bench(torch, 5)}))
        return
    if args.only == "decode":
        # decode-sized lookups with cached packed keys (mpl_lookup alone): the
        # 67,108,864-slot table at 1, 16 and 64 tokens, and the
        # 268,435,456-slot table (n = 16,384, 137 GB) at 64 tokens (the
        # generation workload's lookup), each on a table of every slot
        out = {}
        for n_d, Ms in ((8192, (1, 16, 64)), (16384, (64,))):
            vals = torch.empty((n_d * n_d, 256), dtype=torch.float16, device="cuda")
            hash_normal_(vals, 3, 0.02)
            for M in Ms:
                lkd = Lookup(torch, L, M=M, H=4, n=n_d, d_key=256, d=256, k=16, seed=10 + M, values=vals,
                             rotate=large_rotation(M) if n_d == 8192 else 4)
                lkd.pack()
                out[f"n{n_d}_M{M}"] = {"cached_keys_ms_per_step": time_loop(torch, lkd.lookup, 50, 5),
                                       "slots": n_d * n_d, "tokens": M}
                del lkd
            del vals
            torch.cuda.empty_cache()
        print(json.dumps({"only": args.only, "decode": out}))
        return
    if args.only == "pool_67M_4096":
        vals = torch.empty((8192 * 8192, 256), dtype=torch.float16, device="cuda")
        hash_normal_(vals, 3, 0.02)  # the hash-defined table: the CPU baseline regenerates its rows
        lk3 = Lookup(torch, L, M=4096, H=4, n=8192, d_key=256, d=256, k=16, seed=4106, values=vals,
                     rotate=large_rotation(4096))
        br3 = kernel_breakdown(torch, lk3, args.steps)
        print(json.dumps({"only": args.only, "rotating_batches": lk3.R, "kernels": br3,
                          "gather_roofline": gather_roofline(torch, lk3, br3, args.steps)}))
        return

    # ---- headline: 262,144 slots, 8,192 tokens per step, successive steps on
    # different token batches (as a layer sees them)
    lk = Lookup(torch, L, M=8192, H=4, n=512, d_key=256, d=256, k=16, seed=0, rotate=HEADLINE_ROTATE)
    ms = time_loop(torch, lk.step, args.steps, args.warmup)
    value = lk.M / (ms * 1e-3)
    br = kernel_breakdown(torch, lk, max(20, args.steps // 2))
    roof, roof_other = dominant_roofline(lk, br)

    # ---- large pool: 67,108,864 fp16 slots (34 GB) held in HBM
    large = None
    if not args.no_large:
        n3 = 8192
        vals = torch.empty((n3 * n3, 256), dtype=torch.float16, device="cuda")
        hash_normal_(vals, 3, 0.02)  # the hash-defined table: the CPU baseline regenerates its rows
        sweep = {}
        for M in (1, 16, 256, 4096):
            lk3 = Lookup(torch, L, M=M, H=4, n=n3, d_key=256, d=256, k=16, seed=10 + M, values=vals,
                         rotate=large_rotation(M))
            it = max(10, args.steps // (4 if M == 4096 else 2))
            ms3 = time_loop(torch, lk3.step, it, max(3, args.warmup // 4))
            entry = {"ms_per_step": ms3, "tokens_per_s": M / (ms3 * 1e-3), "rotating_batches": lk3.R}
            # decode with fixed sub-keys (generation): MemoryPool caches the
            # packed keys per parameter version, so a step is mpl_lookup alone
            entry["cached_keys_ms_per_step"] = time_loop(torch, lk3.lookup, it, 3)
            if M == 4096:
                br3 = kernel_breakdown(torch, lk3, it)
                entry["kernels"] = br3
                entry["gather_roofline"] = gather_roofline(torch, lk3, br3, 4 * it)
                entry["score_topk_roofline"] = roofline_for(lk3, br3, "pool_67M_4096")
            sweep[str(M)] = entry
            del lk3
        del vals
        torch.cuda.empty_cache()
        large = {"workload": "decode lookup, 67,108,864 fp16 slots (34 GB), H=4, d_key=256, k=16, d_value=256; "
                             "calls cycle through rotating_batches token batches",
                 "by_tokens": sweep}

    train = div = fact = None
    if not args.no_train:
        train = {"train_step": train_step_bench(torch, max(5, args.steps // 20)),
                 "sparse_update_zipf": sparse_update_bench(torch, max(10, args.steps // 10))}
        div = key_diversity_bench(torch, max(5, args.steps // 20))
        fact = fact_task_bench(torch, max(5, args.steps // 20))

    generation = None if args.no_generate else generation_bench(torch)
    host = host_file = None
    if not args.no_host:
        host = host_pool_bench(torch, max(5, args.steps // 20))
        host_file = host_pool_file_bench(torch, 5)

    cpu = cpu_more = None
    if not args.no_cpu:
        cpu = cpu_lookup_baseline(args.cpu_seconds, n=512, values_dtype=np.float16,
                                  label="text-study")
        cpu_more = {
            "fact_task_16k_fp32": cpu_lookup_baseline(args.cpu_seconds / 2, n=128, values_dtype=np.float32,
                                                      label="fact-task"),
            "training_262k": cpu_train_baseline(args.cpu_seconds),
            "pool_67M_4096": cpu_lookup_67m_baseline(args.cpu_seconds / 2),
        }
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "text-study memory-layer lookup: 8,192 tokens, 262,144 fp16 slots, H=4, "
                               "d_key=256, n_sub_keys=512, top_k=16, d_value=256",
                   "tokens": 8192, "slots": 262144, "values_dtype": "f16", "score_dtype": "f16 MFMA, f32 accumulate",
                   "parallelism": "single GPU"},
        "roofline": roof,
        "roofline_other_kernel": roof_other,
        "kernels": br,
        "pool_67M": large,
        "training_262k": train,
        "key_diversity_67M": div,
        "fact_task_16k_fp32": fact,
        "generation_268M": generation,
        "host_pool_1M": host,
        "host_pool_file_1M": host_file,
        "cpu_baseline": cpu,
        "cpu_baselines_other": cpu_more,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
