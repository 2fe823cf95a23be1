#!/usr/bin/env python3
"""Benchmark of the paged KV-cache hot path on one MI355X.

Workload (default, configuration 2 -- the Llama-3-8B KV shape): 32 layers, batch 16, 8 KV heads x
128, bf16, page 16.  Every row is prefilled with 512 tokens (untimed), then the configuration's
trajectory is 256 decode steps of the cache: for every layer, append 1 token per row and
materialise the whole contiguous [B, H, seq, D] K and V (ctx 513 -> 768).  `--steps K` times K
consecutive steps of that trajectory: all of it for K >= 256 (the default), else the K steps
centred in it -- reached by running the steps before them untimed after the prefill -- so that
the timed steps move the trajectory's mean bytes per step; the first K steps are reported beside
them (`first_steps`).  Inputs are N(0, 1) in fp32 rounded to the cache dtype from a seeded
generator and already resident in HBM.

`--config 1..5` selects the five benchmark configurations (C1 tiny plumbing, C2 Llama-3-8B
decode, C3 fragmented ragged batch with a random page permutation, C4 32k chunked prefill, C5
80-layer 70B-class share with the pool at 90 % occupancy: before every decode step two seeded
rows are freed and re-prefilled with 8192 new tokens, which take the pages released rows left).

A step runs as one replay of a captured HIP graph of the per-layer fused append+gather launches
(graph mode, C1-C4; the step's new K/V are first copied into the graph's static input buffer,
one copy for K and V, as a model's fused K/V projection would write them; every graph the window
uses is captured before timing), or as host-launched layer calls (eager mode, the per-call path
HF attention takes; C5).
Throughput counts algorithmic bytes per step, summed over layers: append 2*B*T*tb (read new,
write page) + gather sum_b(ctx_b)*tb (read) + B*S_max*tb (write, zero padding of short rows
included), tb = 2*H*D*esize; metadata is not counted.  Per-step bytes come from the same length
arithmetic the kernels apply, run on the host.  C5's re-prefill (2*2*8192*tb per layer: read
new, write pages) is timed and reported on its own (`refill`); its decode updates are bracketed
with HIP events per launch and `value` counts them alone.

`roofline` is the dominant kernel alone: in graph mode the same graphs replayed without the
input copies, timed with HIP events on the stream they run on; in eager mode the event-bracketed
update launches; `achieved` = algorithmic bytes per launch / average launch duration.
`traffic` (measured HBM bytes per launch) is read from the committed rocprof counter summary
profiles/stream_kernel_c<N>_traffic.json when it holds this run's window; otherwise it is null
and `traffic_measured` gives the counter ratio and the window it was measured at.

`cpu_baseline` is the reference CPU path -- the reference layer's per-(row, token) append and its
view + .contiguous() gather, restated in torch (oracle/kv_oracle_torch.py, checked against the
numpy oracle) -- on the host's cores (torch.set_num_threads), over the same input bits and the
GPU's own window (C1/C2: every layer; larger configs: layer 0 over the window's first steps, x L),
timing the decode updates only, step by step: the median step after one warm-up step (`total`
keeps the rate over the summed steps); `numpy_one_thread` beside it (C1/C2) is the numpy oracle on
one core.  The same run checks the
GPU's layer-0 K/V after the window bit for bit against it (`parity`).

`paged_attention` (bf16/fp16 configurations) times the decode-attention kernel that reads K/V
from the pages through the block table (the step the gathered K/V feed), over the pools as the
timed run left them: one call per layer with G query heads per KV head (4, the Llama-3-8B ratio;
8 for the 70B-class C5), captured in a graph and replayed; algorithmic bytes per call = every
visible K and V element once + query + output.  Layer 0 is checked against an fp32 attention over
the gathered K/V.  C2 also reports it at the trajectory's middle (`at_mid_context`: every row
cropped to 650 positions after the first measurement).

`beam_select` times a beam reorder (Cache.reorder_cache) of every layer one decode step past
the prefill: one in-place selection for all layers that shares full pages, moves each taken
row's partial last page and copies it only for repeated rows (graph-replayed; also as the host
call), next to the reference's dense keys[indices] over [B, H, blocks, P, D] per layer on the
same GPU; layer 0 is checked bit for bit against the gathered rows before the selections, and
the pool's sharing invariants are checked.

`quantized_kv` (`--quant`) runs the same prefill and decode steps on fp8 quantised pages
(QuantPagePool: blocks behind a 128-token residual window as E4M3 codes with E8M0 scales),
graph-replayed, and times the dequantising gather alone for its roofline; layer 0 is compared
bit for bit with the quantisation oracle and, for the error quantisation introduces, with the
full-precision K/V.

Prints ONE JSON line.  `--pmc-probe` instead makes, once, the launches the counter and trace runs
profile, as the timed run makes them (graphs in graph mode): the prefill and the steps before the
window, a 64 MiB elementwise pass (the counters' calibration, and the marker after which the
window's launches follow), the window, then one decode-attention call per layer; with `--quant`,
the fp8 leg's prefill, the marker, its decode steps and one dequantising gather per layer.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
CPU_BASELINE_SECONDS = 10.0  # CPU work (timed window and the untimed steps before it) the baseline repeats passes to reach (at most 8)
METRIC = "paged KV append+gather GB/s (% HBM peak); µs per decode-step cache update"
KERNEL = ("stream kernel, fused append + gather, one launch per layer: lean_stream_kernel<8, 2> (1-page tiles; "
          "lean_balanced_kernel<8, 2>, equal unaligned chunks, when their count is not a multiple of the CUs) while "
          "every 1-page tile fits on the CUs at once, lean_stream_kernel<16, 2> (2-page tiles) while those do, else "
          "stream_kernel_rounds<16, 2> (several dispatch rounds, as at C3-C5)")

# prefill: ("uniform", n) | ("ragged", lo, hi, seed) | ("chunks", count, size)
CONFIGS = {
    # C1 runs eager: a graph launch costs the host ~30 us, more than this step's two kernels
    1: dict(name="C1 tiny plumbing", layers=2, batch=1, heads=4, dim=64, page=16, dtype="float32",
            prefill=("uniform", 32), decode=128, seed=1001, mode="eager", cpu_steps=None),
    2: dict(name="C2 Llama-3-8B KV shape", layers=32, batch=16, heads=8, dim=128, page=16, dtype="bfloat16",
            prefill=("uniform", 512), decode=256, seed=1002, mode="graph", cpu_steps=None,
            attention_mid_context=650),
    3: dict(name="C3 fragmented ragged batch", layers=32, batch=64, heads=8, dim=128, page=16, dtype="bfloat16",
            prefill=("ragged", 128, 4096, 2003), perm_seed=3003, decode=128, seed=1003, mode="graph",
            cpu_steps=8),
    4: dict(name="C4 long-context chunked prefill", layers=32, batch=1, heads=8, dim=128, page=32, dtype="float16",
            prefill=("chunks", 16, 2048), decode=64, seed=1004, mode="graph", cpu_steps=16),
    5: dict(name="C5 70B-class single-GPU share", layers=80, batch=32, heads=8, dim=128, page=16, dtype="bfloat16",
            prefill=("uniform", 8192), decode=64, seed=1005, mode="eager", occupancy=0.9,
            churn=(2, 4005), refill=True, cpu_steps=4, group=8),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed decode steps (default: the config's)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed decode steps (default 16, C3-C5: 2)")
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--mode", choices=["graph", "eager"], default=None, help="default: the config's")
    ap.add_argument("--separate-commit", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=None,
                    help="layers the CPU baseline runs (C1/C2 default: all)")
    ap.add_argument("--repeat", type=int, default=None, help="timed repetitions; the best is reported")
    ap.add_argument("--window-start", type=int, default=None,
                    help="first timed decode step (default: the timed steps centred in the trajectory)")
    ap.add_argument("--pmc-probe", action="store_true", help="the profiled launches, once, for rocprof runs")
    ap.add_argument("--no-attention", action="store_true", help="skip the paged decode-attention leg")
    ap.add_argument("--no-beam", action="store_true", help="skip the beam-reorder (select_rows) leg")
    ap.add_argument("--quant", action="store_true", help="add the fp8 quantised-KV leg (not run by default)")
    ap.add_argument("--batch", type=int, default=None,
                    help="rows per layer instead of the config's (small-launch characterisation, e.g. --batch 1)")
    ap.add_argument("--bucket", type=int, default=None,
                    help="graph extent bucket in positions (default: the step's own; 0: one graph over the capacity)")
    return ap.parse_args()


def elem_size(cfg):
    return {"float32": 4, "bfloat16": 2, "float16": 2, "float64": 8}[cfg["dtype"]]


def tok_bytes(cfg):
    return 2 * cfg["heads"] * cfg["dim"] * elem_size(cfg)


def prefill_lengths(cfg):
    """Per-row context after the prefill."""
    import numpy as np

    kind = cfg["prefill"]
    B = cfg["batch"]
    if kind[0] == "uniform":
        return [kind[1]] * B
    if kind[0] == "ragged":  # longest rows first: the reference API appends to rows [0, batch)
        rng = np.random.default_rng(kind[3])
        return sorted(rng.integers(kind[1], kind[2] + 1, size=B).tolist(), reverse=True)
    return [kind[1] * kind[2]] * B


def prefill_calls(cfg):
    """(batch, tokens, gather_after) of the prefill's append calls, in order."""
    kind = cfg["prefill"]
    if kind[0] == "uniform":
        return [(cfg["batch"], kind[1], True)]
    if kind[0] == "chunks":
        return [(cfg["batch"], kind[2], True)] * kind[1]
    lens = prefill_lengths(cfg)
    calls, done = [], 0
    for b in range(len(lens), 0, -1):
        need = lens[b - 1] - done
        if need > 0:
            calls.append((b, need, False))
            done += need
    return calls


def churn_rows(cfg, steps):
    """Rows freed (and, with `refill`, re-prefilled) before each decode step."""
    import numpy as np

    if "churn" not in cfg:
        return [[] for _ in range(steps)]
    n, seed = cfg["churn"]
    rng = np.random.default_rng(seed)
    return [sorted(rng.choice(cfg["batch"], size=n, replace=False).tolist()) for _ in range(steps)]


def step_bytes_all(cfg, steps, churn):
    """Algorithmic bytes of each decode step's updates (all layers), from the host length
    arithmetic; churned rows restart empty, or at their prefill length when re-prefilled."""
    start = prefill_lengths(cfg)
    lens = list(start)
    tb, B, L = tok_bytes(cfg), cfg["batch"], cfg["layers"]
    out = []
    for s in range(steps):
        for r in churn[s]:
            lens[r] = start[r] if cfg.get("refill") else 0
        lens = [x + 1 for x in lens]
        out.append(L * (2 * B * tb + sum(lens) * tb + B * max(lens) * tb))
    return out


def longest_rows(cfg, steps, churn):
    """Longest row after each decode step's append (the extent its graph covers)."""
    start = prefill_lengths(cfg)
    lens = list(start)
    out = []
    for s in range(steps):
        for r in churn[s]:
            lens[r] = start[r] if cfg.get("refill") else 0
        lens = [x + 1 for x in lens]
        out.append(max(lens))
    return out


def window_start(cfg, steps):
    """First decode step of the timed window: the `steps` steps centred in the configuration's
    trajectory when they are fewer (their bytes per step are then its mean), else step 0."""
    total = cfg["decode"]
    return (total - steps) // 2 if steps < total else 0


def host_threads():
    """Threads of the CPU baseline: the cores this process may run on, capped by
    OMP_NUM_THREADS when it is set (the GPU box sets it to its CPU share)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_baseline(cfg, wl, start, steps, layers):
    """The reference CPU path (oracle/kv_oracle_torch.py) on the host's cores, timed as the
    measurement plan says: `layers` layers, each prefilled untimed and run through the steps
    before the window untimed, then one warm-up step (the step before the window; when the window
    starts at step 0, its first step, which the median then leaves out) and the GPU's own window
    of decode steps [start, start + steps) timed one step at a time with the host clock (churned
    rows are freed and re-prefilled between steps, untimed).  A step's time is the sum over the
    layers (times L / layers when fewer layers run); `ms_per_step` is the median over the
    window's steps, pooled over passes (passes repeat the layers until about CPU_BASELINE_SECONDS
    of work, at most 8).  `total` keeps the rate over every timed step (bytes over summed time).
    Returns (result, layer-0 K/V after the window, as torch tensors).  For C1/C2 the numpy oracle
    on one core times layer 0 beside it the same way."""
    import numpy as np
    import torch

    from oracle.kv_oracle import DenseLayerOracle
    from oracle.kv_oracle_torch import DenseLayerTorch

    B, P, L = cfg["batch"], cfg["page"], cfg["layers"]
    cap = max(prefill_lengths(cfg)) + wl.n_steps
    refill = tuple(t.cpu() for t in wl.refill) if wl.refill is not None else None
    n = start + steps
    warm = 1 if start == 0 else 0  # the window's first step is the warm-up when nothing precedes it
    threads = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)

    def timed_layer(ref, layer, to_input):
        """Per-step seconds of steps [start, n) of one layer, and its last output."""
        for k, v in wl.prefill_inputs(layer):
            ref.append(to_input(k), to_input(v))
        kd = [to_input(wl.k_dec[s, layer]) for s in range(n)]
        vd = [to_input(wl.v_dec[s, layer]) for s in range(n)]
        spent, out = np.zeros(steps), None
        for s in range(n):
            rows = wl.churn[s]
            if rows:
                ref.release_rows(rows)
                if refill is not None:
                    ref.append_rows(rows, to_input(refill[0]), to_input(refill[1]))
            t0 = time.perf_counter()
            out = ref.update(kd[s], vd[s])
            if s >= start:
                spent[s - start] = time.perf_counter() - t0
        return spent, out

    def summarise(per_pass):
        """(median seconds per step over the pooled window steps, summed seconds) for per-pass arrays
        of per-step seconds over the layers run."""
        pooled = np.concatenate([p[warm:] for p in per_pass]) * (L / layers)
        return float(np.median(pooled)), float(sum(p.sum() for p in per_pass))

    try:
        per_pass, final, passes, wall0 = [], None, 0, time.perf_counter()
        while passes < 8 and (passes == 0 or time.perf_counter() - wall0 < CPU_BASELINE_SECONDS):
            step_s = np.zeros(steps)
            for layer in range(layers):
                spent, out = timed_layer(DenseLayerTorch(B, cap, P), layer, lambda t: t.cpu())
                step_s += spent
                if layer == 0 and passes == 0:
                    final = out
            per_pass.append(step_s)
            passes += 1
    finally:
        torch.set_num_threads(prev)
    med, total = summarise(per_pass)
    window_bytes = np.asarray(wl.step_bytes[start:n], dtype=np.float64)
    step_bytes = float(window_bytes[warm:].mean()) if steps > warm else float(window_bytes.mean())
    result = {
        "value": round(step_bytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"decode steps {start}..{n - 1} (the GPU's timed window; append 1 token x {B} rows + materialised "
                  f"gather), {layers} of {L} layers" + ("" if layers == L else f" (x{L // layers} extrapolated)")
                  + f", median step of {passes} pass(es) after one warm-up step; torch restatement of the reference "
                  f"kv_cache.py _python_append + current_tensors (view + .contiguous()) on {threads} threads; "
                  f"same input bits",
        "ms_per_step": round(med * 1e3, 3),
        "total": {"value": round(float(window_bytes.sum()) * layers / L * passes / total / 1e9, 3),
                  "seconds": round(total, 2),
                  "note": "every timed step of every pass: window bytes over summed step time"},
    }
    if cfg["cpu_steps"] is None:  # C1/C2: the numpy oracle on one core, layer 0
        from kvgen import to_bits

        spent, _ = timed_layer(DenseLayerOracle(B, cap, P), 0, to_bits)
        med1 = float(np.median(spent[warm:] if steps > warm else spent)) * L
        result["numpy_one_thread"] = {"value": round(step_bytes / med1 / 1e9, 3), "cores": 1,
                                      "ms_per_step": round(med1 * 1e3, 3),
                                      "sample": f"layer 0 x decode steps {start}..{n - 1} (x{L} layers), median step, "
                                                f"numpy oracle"}
    return result, final


class Workload:
    """Pools, prefill, per-step inputs and churn of one configuration on cuda:0, for decode steps
    [0, n_steps) of its trajectory."""

    def __init__(self, cfg, n_steps, dev):
        import numpy as np
        import torch

        from barqtrain_amd.paged import PagePool

        self.cfg, self.dev = cfg, dev
        self.dtype = getattr(torch, cfg["dtype"])
        L, B, H, D, P = cfg["layers"], cfg["batch"], cfg["heads"], cfg["dim"], cfg["page"]
        self.n_steps = n_steps
        self.steps_cap = n_steps
        lens = prefill_lengths(cfg)
        cap = max(lens) + n_steps
        mb = math.ceil(cap / P)
        num_pages = B * mb
        if "occupancy" in cfg:  # the prefill's pages fill `occupancy` of the pool
            live = sum(math.ceil(x / P) for x in lens)
            num_pages = max(math.ceil(live / cfg["occupancy"]), live + B * math.ceil(n_steps / P) + B)
        order = None
        if "perm_seed" in cfg:
            perm = np.random.default_rng(cfg["perm_seed"]).permutation(num_pages).astype(np.int32)
            order = torch.from_numpy(perm).to(dev)
        self.order = order
        self.pools = [PagePool(max_batch=B, max_blocks=mb, page_size=P, kv_heads=H, head_dim=D, dtype=self.dtype,
                               device=dev, num_pages=num_pages, page_order=order) for _ in range(L)]
        gen = torch.Generator(device=dev).manual_seed(cfg["seed"])
        # K and V of every decode step in one buffer, [step, K|V, L, B, H, 1, D] (a model's fused
        # projection writes both): a step's inputs arrive with one copy
        kv = torch.empty((n_steps, 2, L, B, 1, H, D), dtype=self.dtype, device=dev)
        kv[:, 0] = self._normal(gen, (n_steps, L, B, 1, H, D))
        kv[:, 1] = self._normal(gen, (n_steps, L, B, 1, H, D))
        self.kv_dec = kv.transpose(4, 5)
        self.k_dec = self.kv_dec[:, 0]
        self.v_dec = self.kv_dec[:, 1]
        self.churn = churn_rows(cfg, n_steps)
        self.step_bytes = step_bytes_all(cfg, n_steps, self.churn)
        self.longest = longest_rows(cfg, n_steps, self.churn)
        self.refill = None
        if cfg.get("refill"):  # one seeded prefill that every re-prefilled row takes
            n, ctx = cfg["churn"][0], lens[0]
            g = torch.Generator(device=dev).manual_seed(cfg["seed"] + 7)
            self.refill = (self._normal(g, (n, ctx, H, D)).transpose(1, 2),
                           self._normal(g, (n, ctx, H, D)).transpose(1, 2))
            self.refill_bytes = L * 2 * n * ctx * tok_bytes(cfg)  # per step: read new + write pages

    def _normal(self, gen, shape):
        import torch

        return torch.randn(shape, generator=gen, device=self.dev, dtype=torch.float32).to(self.dtype)

    def prefill_inputs(self, layer):
        """The prefill's (K, V) per append call of `layer`, HF layout [b, H, t, D] (physical
        [b, t, H, D]); regenerated identically on every call from a per-layer seed."""
        import torch

        cfg = self.cfg
        gen = torch.Generator(device=self.dev).manual_seed(cfg["seed"] * 1000 + layer)
        for b, t, _ in prefill_calls(cfg):
            shape = (b, t, cfg["heads"], cfg["dim"])
            yield self._normal(gen, shape).transpose(1, 2), self._normal(gen, shape).transpose(1, 2)

    def prefill(self):
        for layer, pool in enumerate(self.pools):
            pool.reset(self.order)
            for (b, t, gather), (k, v) in zip(prefill_calls(self.cfg), self.prefill_inputs(layer)):
                if gather:
                    pool.update(k, v)
                else:
                    pool.append(k, v)

    def churn_layer(self, s, pool):
        """Step s's churn on one layer: its rows freed and, with `refill`, re-prefilled."""
        rows = self.churn[s]
        if rows:
            pool.free_rows(rows)
            if self.refill is not None:
                pool.append_rows(rows, *self.refill)


def pair_kernel_bounds(pairs, max_seq, rows, quantised, cus=256):
    """Whether the library takes a one-token decode call in one launch (its pair kernel), as its
    host code decides (barq_kv_attention.hip, launch_typed): up to 8 query rows; at most 44
    16-position chunks, or, from 128 (row, kv head) pairs with up to 4 query rows, 64 (over
    two-byte pages 128 from 256 pairs); with three or more 8-wave workgroups a pair resident (one a
    CU), up to 24 chunks a workgroup (at most 8 of them, within one 256-block window), else up to
    72 a workgroup over at most 32 of them."""
    if pairs < 1 or rows > 8:
        return False
    chunks = -(-max_seq // 16)
    part = 11 if rows <= 4 else 14
    nsplit = min(8, cus // pairs) if pairs <= 512 and chunks >= 2 * part else 1
    if rows > 4 or pairs < 128:
        bound = 44
    else:
        bound = 128 if pairs >= 256 and not quantised else 64
    if nsplit > 2:
        bound = min(256, max(bound, nsplit * 24))
    if chunks <= bound:
        return True
    nlong = min(32, cus // pairs) if pairs <= 512 else 0
    return nlong > 2 and chunks <= nlong * 72


def attention_leg(cfg, pools, B, dev, reps=20, kv_bytes=None, probe=False):
    """Decode attention over the pools' current rows: one launch per layer, graph-replayed.
    kv_bytes(pool, lens): the K/V bytes one call reads (default: every visible element in the
    cache dtype).  `probe`: one eager call per layer, nothing timed (for counter runs)."""
    import numpy as np
    import torch

    from barqtrain_amd.paged import _gpu_backend

    backend = _gpu_backend()
    H, D, L = cfg["heads"], cfg["dim"], len(pools)
    G = cfg.get("group", 4)
    dtype = pools[0].dtype
    esize = torch.empty(0, dtype=dtype).element_size()
    gen = torch.Generator(device=dev).manual_seed(cfg["seed"] + 17)
    q = torch.randn((B, G * H, 1, D), generator=gen, device=dev).to(dtype)
    scale = D ** -0.5
    lens = [np.asarray(p.lens[:B]).copy() for p in pools]
    max_seq = max(int(x.max()) for x in lens)
    outs = [torch.empty((B, 1, G * H, D), dtype=dtype, device=dev).transpose(1, 2) for _ in pools]
    wss = [p.attention_workspace(backend.attention_workspace_bytes(p.tensors, B, G * H, 1, max_seq, 0))
           for p in pools]

    def step():
        for layer, pool in enumerate(pools):
            pool._attention_call(backend, q, outs[layer], scale, max_seq, 0, wss[layer])

    step()
    torch.cuda.synchronize()
    io = 2 * B * G * H * D * esize  # query read + output written
    if kv_bytes is None:
        call_bytes = [int(x.sum()) * H * D * 2 * esize + io for x in lens]
    else:
        call_bytes = [kv_bytes(p, x) + io for p, x in zip(pools, lens)]
    if probe:
        return {"attention_calls": L, "attention_algorithmic_bytes_per_call": int(sum(call_bytes) / L),
                "attention_context": f"{int(min(x.min() for x in lens))}..{max_seq}"}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    graph.replay()
    torch.cuda.synchronize()
    best = None
    for _ in range(3):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / reps
        best = ms if best is None else min(best, ms)
    per_call_us = best * 1e3 / L
    gbs = sum(call_bytes) / (best / 1e3) / 1e9
    # layer 0 against an fp32 attention over the gathered K/V (rows 0 and B - 1)
    k, v = pools[0].gather(B)
    tol = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    err, ok = 0.0, True
    for b in sorted({0, B - 1}):
        n = int(lens[0][b])
        kk = k[b, :, :n].float().repeat_interleave(G, 0)
        vv = v[b, :, :n].float().repeat_interleave(G, 0)
        sc = torch.matmul(q[b].float(), kk.transpose(1, 2).contiguous()) * scale
        ref = torch.matmul(torch.softmax(sc, -1), vv)
        diff = (outs[0][b].float() - ref).abs()
        err = max(err, diff.max().item())
        ok = ok and bool((diff <= tol * ref.abs() + 2e-5).all().item())
    torch.cuda.synchronize()
    if any(p.errors() for p in pools):
        raise SystemExit("device error bits set by the attention leg")
    gathered = 3 * (sum(call_bytes) - L * io) / L  # gather reads + writes K/V, attention re-reads
    cold = "<..., COLD> (fp8 pages read as codes)" if getattr(pools[0], "quantized", False) else ""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    if pair_kernel_bounds(B * H, max_seq, G, bool(cold), cus):
        kname = "attention_pair_kernel" + cold + " (one launch per layer)"
    else:
        kname = "attention_flat_kernel" + cold + " + attention_merge_kernel (one launch pair per layer)"
    return {
        "kernel": kname,
        "query_heads_per_kv_head": G,
        "us_per_layer_call": round(per_call_us, 2),
        "us_per_step_all_layers": round(best * 1e3, 1),
        "achieved": round(gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(gbs / HBM_PEAK_GBS, 4),
        "bytes_per_call": int(sum(call_bytes) / L),
        "context": f"{int(min(x.min() for x in lens))}..{max_seq}",
        "gathered_path_bytes_per_call": int(gathered),
        "parity": {"layer0_max_abs_err_vs_fp32": round(err, 6), "tolerance": f"{tol:g} x |ref| + 2e-5",
                   "ok": ok},
    }


def beam_leg(cfg, wl, dev, reps=20):
    """Beam reorder (Cache.reorder_cache / batch_select_indices) of every layer, one decode step
    past the prefill so that every row ends in a partial page: one selection for all layers in one
    set of launches (barq_kv_select_rows_layers), timed as a graph replay (device time) and as the
    host call select_rows_layers; beside it, the reference's own operation on the same GPU --
    keys[indices] / values[indices] over the dense [B, H, blocks, P, D] cache of every layer
    (kv_cache.py:175-183), timed on one layer and scaled by the layer count."""
    import numpy as np
    import torch

    from barqtrain_amd.paged import _gpu_backend, _pool_group, select_rows_layers
    from capi_pool import check_pool_invariants

    backend = _gpu_backend()
    pools = wl.pools
    L, B, H, D, P = cfg["layers"], cfg["batch"], cfg["heads"], cfg["dim"], cfg["page"]
    wl.prefill()
    for layer, pool in enumerate(pools):
        pool.update(wl.k_dec[0, layer], wl.v_dec[0, layer])
    torch.cuda.synchronize()
    rows = sorted(np.random.default_rng(cfg["seed"] + 29).integers(0, B, size=B).tolist())
    k0, v0 = (t.clone() for t in pools[0].gather(B))
    r = np.asarray(rows)
    copies = int(pools[0].tail_block_counts(r)[pools[0].repeated_mask(r)].sum())
    page_bytes = P * H * D * pools[0].dtype.itemsize
    sel_bytes = copies * page_bytes * 2 * 2  # K and V pages, read + written

    select_rows_layers(pools, rows)  # warm (pinned index buffer, pool group, workspace)
    torch.cuda.synchronize()
    host_best = None
    for _ in range(5):
        t0 = time.perf_counter()
        select_rows_layers(pools, rows)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        host_best = dt if host_best is None else min(host_best, dt)
    entry = _pool_group(pools)
    idx = torch.tensor(rows, dtype=torch.int32, device=dev)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        backend.pool_group_select_rows_(entry["group"], idx, entry["ws"])
    graph.replay()
    torch.cuda.synchronize()
    applied = 6 + 1  # host calls 6, warm replay 1
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    graph_ms = start.elapsed_time(end) / reps
    applied += reps
    if any(p.errors() for p in pools):
        raise SystemExit("device error bits set by the beam leg")
    order = np.arange(B)
    for _ in range(applied):
        order = order[r]
    sel = torch.as_tensor(order, device=dev)
    k1, v1 = pools[0].gather(B, k0.shape[2])  # the host shadow lags the graph replays
    ok = bool(torch.equal(k1.view(torch.int16), k0[sel].view(torch.int16))
              and torch.equal(v1.view(torch.int16), v0[sel].view(torch.int16)))
    pool = pools[0]
    check_pool_invariants(pool.block_table.cpu().numpy(), pool.seq_lens.cpu().numpy(),
                          pool.high_water.cpu().numpy(), pool.free_pages.cpu().numpy(),
                          pool.ctrl.cpu().numpy(), pool.page_shares.cpu().numpy(), P)
    held = pool.num_pages - int(pool.ctrl[0].item())

    mb = pool.max_blocks
    kd = torch.empty((B, H, mb, P, D), dtype=pool.dtype, device=dev)
    vd = torch.empty_like(kd)
    ko, vo = torch.empty_like(kd), torch.empty_like(vd)
    lidx = idx.long()

    def dense():
        torch.index_select(kd, 0, lidx, out=ko)
        torch.index_select(vd, 0, lidx, out=vo)

    dense()
    dgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(dgraph):
        dense()
    dgraph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        dgraph.replay()
    end.record()
    torch.cuda.synchronize()
    dense_ms = start.elapsed_time(end) / reps
    dense_bytes = 2 * 2 * kd.numel() * kd.element_size()
    del kd, vd, ko, vo
    sets = -(-L // 32)
    return {
        "kernels": f"select_plan_kernel + select_build_kernel + select_settle_kernel, {sets} set(s) of "
                   f"launches for {L} layers",
        "selection": f"{B} rows from sorted seeded parents ({len(set(rows))} distinct), context "
                     f"{int(pool.lens[:B].min())}..{int(pool.lens[:B].max())}",
        "us_per_step_all_layers": round(graph_ms * 1e3, 1),
        "host_us_per_step_all_layers": round(host_best * 1e6, 1),
        "pages_copied_per_layer": copies,
        "bytes_copied_per_layer": sel_bytes,
        "pages_held_layer0": held,
        "reference_dense_index_us_per_step": round(dense_ms * 1e3 * L, 1),
        "reference_dense_bytes_per_layer": dense_bytes,
        "speedup_vs_reference_dense": round(dense_ms * L / graph_ms, 1),
        "parity": {"layer0_bit_exact_after_selections": ok, "selections_applied": applied,
                   "invariants_checked": True},
    }


def quant_leg(cfg, wl, steps, dev, bf16_ms_per_step, window=128, reps=10, probe=None):
    """fp8 quantised pages (QuantPagePool): every layer prefilled as the configuration does (long
    appends in 256-token chunks, each followed by quantisation), then `steps` decode steps of
    append + quantise-what-left-the-window + dequantising gather, graph-replayed; no row churn.
    The dequantising gather alone is timed from a graph of its launches (the dominant kernel's
    roofline); layer 0 is compared with the oracle after the steps, and with the full-precision
    K/V of the main run for the error the quantisation introduces."""
    import numpy as np
    import torch

    from barqtrain_amd.graph import CapturedDecodeStep
    from barqtrain_amd.paged import QuantPagePool, _gpu_backend
    from kvgen import to_bits
    from oracle.kv_quant_oracle import QuantLayerOracle

    backend = _gpu_backend()
    L, B, H, D, P = cfg["layers"], cfg["batch"], cfg["heads"], cfg["dim"], cfg["page"]
    cap = max(prefill_lengths(cfg)) + wl.steps_cap
    mb = math.ceil(cap / P)
    # no beam selection here: the hot pool holds the window and a prefill chunk per row, without
    # the default's room for selection copies
    hot = B * (-(-(window + 64) // P) + 2)
    pools = [QuantPagePool(max_batch=B, max_blocks=mb, page_size=P, kv_heads=H, head_dim=D, dtype=wl.dtype,
                           device=dev, window=window, num_pages=hot) for _ in range(L)]
    kvin = torch.empty((2, L, B, H, 1, D), dtype=wl.dtype, device=dev)
    step = CapturedDecodeStep(pools, B, 1, inputs=(kvin[0], kvin[1]))

    def prefill():
        for layer, pool in enumerate(pools):
            pool.reset()
            for k, v in wl.prefill_inputs(layer):
                pool.append(k, v)

    def run(s):
        kvin.copy_(wl.kv_dec[s])
        step.replay(views=False)

    tb, esize = tok_bytes(cfg), elem_size(cfg)

    def cold_read_bytes(lens_b, cold_b):
        """Bytes a dequantising read of rows with these lengths and quantised blocks fetches."""
        c = np.minimum(cold_b * P, lens_b)
        return int((lens_b - c).sum() * tb + c.sum() * 2 * H * D + (c // P).sum() * (H * D + P * H))

    if probe is not None:  # counter runs: prefill, marker, the decode steps, one gather per layer
        prefill()
        step.prepare([max(prefill_lengths(cfg)) + s + 1 for s in range(steps)])
        lens0 = pools[0].lens[:B].astype(np.int64).copy()
        probe()
        update_bytes = []
        for s in range(steps):
            run(s)
            if s % 16 == 15:
                torch.cuda.synchronize()
                print(f"pmc-probe: fp8 step {s} done", file=sys.stderr, flush=True)
            lens_s = lens0 + s + 1
            cold_s = np.maximum(lens_s - window, 0) // P
            update_bytes.append(2 * B * tb + cold_read_bytes(lens_s, cold_s) + B * int(lens_s.max()) * tb)
        seq = pools[0].max_len(B)
        ko, vo = pools[0]._new_out(B, seq)
        for pool in pools:
            backend.pool_gather_cold(pool.tensors, pool.cold_tensors, pool.window, ko, vo, B, seq, 0)
        torch.cuda.synchronize()
        lens_e = pools[0].lens[:B].astype(np.int64)
        gather_bytes = cold_read_bytes(lens_e, pools[0].cold_blocks[:B].astype(np.int64)) + B * seq * tb
        attn_info = {}
        if D == 128 and P % 16 == 0:  # one decode attention per layer over the quantised pages
            def attn_bytes(pool, lens_b):
                return cold_read_bytes(lens_b, pool.cold_blocks[:B].astype(np.int64))

            attn_info = attention_leg(cfg, pools, B, dev, reps=1, kv_bytes=attn_bytes, probe=True)
            print("pmc-probe: fp8 attention done", file=sys.stderr, flush=True)
        print(json.dumps({"pmc_probe": "quant", "config": cfg["name"], "steps": steps, "launches": steps * L,
                          "update_algorithmic_bytes_per_launch": float(np.mean(update_bytes)),
                          "gather_calls": L, "gather_algorithmic_bytes_per_launch": gather_bytes,
                          "context": f"{int(lens0.min()) + 1}..{int(lens_e.max())}", **attn_info}), flush=True)
        return None
    prefill()
    # every graph the steps replay (each extent bucket, with and without the compress launch)
    # captured before the timed region
    step.prepare([max(prefill_lengths(cfg)) + s + 1 for s in range(steps)])
    for s in range(min(4, steps)):
        run(s)
    torch.cuda.synchronize()
    prefill()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for s in range(steps):
        run(s)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    if any(p.errors() for p in pools):
        raise SystemExit("device error bits set by the quantised-KV leg")

    # the dequantising gather alone, over the final state
    seq = pools[0].max_len(B)
    outs = [pools[0]._new_out(B, seq) for _ in range(2)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i, pool in enumerate(pools):
            ko, vo = outs[i % 2]
            backend.pool_gather_cold(pool.tensors, pool.cold_tensors, pool.window, ko, vo, B, seq, 0)
    graph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    gather_us = start.elapsed_time(end) * 1e3 / reps / L
    lens = pools[0].lens[:B].astype(np.int64)
    cold = pools[0].cold_blocks[:B].astype(np.int64)
    cold_tok = cold * P
    hot_tok = lens - cold_tok
    gather_bytes = int(hot_tok.sum() * tb + cold_tok.sum() * 2 * H * D       # hot pages, codes
                       + cold.sum() * (H * D + P * H)                          # scales
                       + B * seq * tb)                                         # output
    gbs = gather_bytes / (gather_us * 1e-6) / 1e9

    # parity: layer 0 against the oracle fed the same inputs
    oracle = QuantLayerOracle(B, cap, P, window, {"bfloat16": "bf16", "float16": "f16"}[cfg["dtype"]])
    for k, v in wl.prefill_inputs(0):
        oracle.append(to_bits(k), to_bits(v))
    for s in range(steps):
        oracle.append(to_bits(wl.k_dec[s, 0]), to_bits(wl.v_dec[s, 0]))
    gk, gv = pools[0].gather(B)
    ok, ov = oracle.current_tensors()
    bit_exact = bool(np.array_equal(to_bits(gk), ok) and np.array_equal(to_bits(gv), ov))
    # error against full precision: the main run's pools hold the same tokens (no churn configs)
    err = None
    if not any(wl.churn[:steps]):
        exact = wl.pools[0]
        exact.reset(wl.order)
        for k, v in wl.prefill_inputs(0):
            exact.append(k, v)
        for s in range(steps):
            exact.append(wl.k_dec[s, 0], wl.v_dec[s, 0])
        xk, xv = exact.gather(B)
        err = {}
        for name, g, x in (("key", gk, xk), ("value", gv, xv)):
            d = (g.float() - x.float())
            err[name] = {"rms_rel": round(float(d.pow(2).mean().sqrt() / x.float().pow(2).mean().sqrt()), 5),
                         "max_abs": round(float(d.abs().max()), 4)}
    def kv_bytes(pool, lens_b):
        c = np.minimum(pool.cold_blocks[:B] * P, lens_b)
        return int((lens_b - c).sum() * H * D * 2 * esize + c.sum() * H * D * 2
                   + (c // P).sum() * (H * D + P * H))

    attn = attention_leg(cfg, pools, B, dev, kv_bytes=kv_bytes) if D == 128 and P % 16 == 0 else None
    mem = pools[0].memory_bytes()
    full = 2 * B * mb * P * H * D * esize
    return {
        "kernels": ("update_cold_lanes_kernel (append + dequantising gather, one launch) per layer, and "
                    "compress_regs_kernel when blocks leave the window; graph-replayed"),
        "format": f"fp8 E4M3 codes, E8M0 scales (keys per channel, values per token over a page), "
                  f"residual window {window} tokens",
        "us_per_step_all_layers": round(ms * 1e3, 1),
        "full_precision_us_per_step": round(bf16_ms_per_step * 1e3, 1),
        "gather_cold_kernel": {"kernel": "gather_cold_lanes_kernel (the dequantising gather alone)",
                               "avg_launch_us": round(gather_us, 2), "bytes_per_launch": gather_bytes,
                               "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                               "frac": round(gbs / HBM_PEAK_GBS, 4)},
        "memory_per_layer_bytes": {**mem, "full_precision_pool": full,
                                   "ratio": round((mem["hot_pages"] + mem["cold_store"]) / full, 3)},
        "context": f"{int(lens.min())}..{int(lens.max())}, quantised blocks per row {int(cold.min())}..{int(cold.max())}",
        "parity": {"layer0_bit_exact_vs_oracle": bit_exact, "after_decode_steps": steps},
        "error_vs_full_precision": err,
        "paged_attention_fp8": attn,
    }


def calibration_pass(dev):
    """64 MiB read + 64 MiB written by one elementwise kernel, three times: the counters' scale,
    and the marker after which a probe's window follows."""
    import torch

    torch.cuda.synchronize()
    src = torch.zeros(64 * 2**20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()


def pmc_probe(cfg, wl, start, steps, run_step, dev, quant):
    """The launches the counter runs profile, as the timed run makes them: the prefill and the
    steps before the window, the calibration pass, the window's steps, then one decode-attention
    call per layer over the state they leave (bf16/fp16, head_dim 128).  With `quant`, the fp8
    leg's prefill, the calibration pass, then its decode steps and one dequantising gather and
    attention call per layer."""
    import torch

    L = cfg["layers"]
    if quant:
        quant_leg(cfg, wl, steps, dev, 0.0, probe=lambda: calibration_pass(dev))
        return
    def progress(what, s):
        # A counter run serialises every dispatch and reads the counters after each one, so a
        # long probe is slow, not hung: a line every 16 steps (after the GPU has finished them)
        # shows how far it got.
        if s % 16 == 15:
            torch.cuda.synchronize()
            print(f"pmc-probe: {what} step {s} done", file=sys.stderr, flush=True)

    wl.prefill()
    print("pmc-probe: prefill enqueued", file=sys.stderr, flush=True)
    for s in range(start):
        run_step(s)
        progress("pre-window", s)
    calibration_pass(dev)
    for s in range(start, start + steps):
        run_step(s)
        progress("window", s)
    torch.cuda.synchronize()
    print("pmc-probe: window done", file=sys.stderr, flush=True)
    attn = cfg["dtype"] in ("bfloat16", "float16") and cfg["dim"] == 128
    attn_info = attention_leg(cfg, wl.pools, cfg["batch"], dev, reps=1, probe=True) if attn else {}
    total = sum(wl.step_bytes[start:start + steps])
    print(json.dumps({"pmc_probe": True, "config": cfg["name"], "window_start": start, "steps": steps,
                      "launches": steps * L, "algorithmic_bytes_per_launch": total / (steps * L),
                      "attention_calls": L if attn else 0, **attn_info}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1. The cache path "
                                   "would shard by sequence, KV head or layer, with no collective on it."}))
        sys.exit(2)
    import torch

    from barqtrain_amd import _ffi
    from barqtrain_amd.graph import CapturedDecodeStep
    from barqtrain_amd.paged import SEPARATE_FINALIZE

    backend = _ffi.load_cuda_backend()
    if backend is None:
        raise SystemExit("barqtrain_cuda HIP backend not built (python -m barqtrain_amd.build)")
    torch.cuda.set_device(0)
    cfg = CONFIGS[args.config]
    if args.batch is not None:
        if args.batch < 1 or "churn" in cfg or cfg["prefill"][0] != "uniform":
            raise SystemExit("--batch takes a positive row count, for configurations with a uniform prefill")
        cfg = dict(cfg, batch=args.batch, name=f"{cfg['name']} (batch {args.batch})")
    steps = args.steps if args.steps is not None else cfg["decode"]
    big = args.config >= 3
    warmup = args.warmup if args.warmup is not None else (2 if big else 16)
    repeat = args.repeat if args.repeat is not None else (1 if big else 3)
    mode = args.mode or cfg["mode"]
    start = window_start(cfg, steps) if args.window_start is None else args.window_start
    if args.window_start is not None and (start < 0 or start + steps > cfg["decode"]):
        raise SystemExit(f"window {start}..{start + steps - 1} is outside the {cfg['decode']}-step trajectory")
    L, B, H, D, P = cfg["layers"], cfg["batch"], cfg["heads"], cfg["dim"], cfg["page"]
    dev = torch.device("cuda", 0)
    wl = Workload(cfg, start + max(steps, warmup), dev)
    pools = wl.pools
    flags = SEPARATE_FINALIZE if args.separate_commit else 0

    graph = None
    last = {}
    marks = []  # eager mode: (start, end) events around every update launch of the window
    if mode == "graph":
        if any(wl.churn):
            raise SystemExit("graph mode replays a fixed step; configurations with row churn run eager")
        kvin = torch.empty((2, L, B, H, 1, D), dtype=wl.dtype, device=dev)
        graph = CapturedDecodeStep(pools, B, 1, separate_commit=args.separate_commit,
                                   inputs=(kvin[0], kvin[1]), bucket=args.bucket)
        graph.prepare(wl.longest)  # no capture inside a timed region

        def run_step(s, record=False):
            kvin.copy_(wl.kv_dec[s])
            graph.replay(views=False)
    else:
        # each step's per-layer input views, made before any timing (a model's projections
        # hand them over ready)
        views = [[(wl.k_dec[s, layer], wl.v_dec[s, layer]) for layer in range(L)] for s in range(wl.n_steps)]

        def run_step(s, record=False):
            churned = bool(wl.churn[s])
            for layer, pool in enumerate(pools):
                if churned:
                    wl.churn_layer(s, pool)
                if record:
                    e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                    e[0].record()
                k, v = views[s][layer]
                out = pool.update(k, v, flags=flags)
                if record:
                    e[1].record()
                    marks.append(e)
                if layer == 0:
                    last["out"] = out

    if args.pmc_probe:
        pmc_probe(cfg, wl, start, steps, run_step, dev, args.quant)
        return

    # The prefill (untimed for the decode metric; reported on its own for chunked prefill), then
    # warm-up steps at the window.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    wl.prefill()
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    for s in range(start + warmup):
        run_step(s)
    torch.cuda.synchronize()

    def timed(fn, lo, n):
        """Best of `repeat`: prefill, steps [0, lo) untimed, then steps [lo, lo + n) bracketed by
        synchronisations and timed with events.  Returns (ms, event-bracketed update ms)."""
        best = None
        for _ in range(max(1, repeat)):
            wl.prefill()
            for s in range(lo):
                fn(s)
            torch.cuda.synchronize()
            marks.clear()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for s in range(lo, lo + n):
                fn(s, record=True) if fn is run_step else fn(s)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1)
            upd = sum(a.elapsed_time(b) for a, b in marks) if marks else None
            if best is None or ms < best[0]:
                best = (ms, upd)
        return best

    # The dominant kernel alone: in graph mode the per-layer launches without the input copies,
    # timed on the stream they run on (the inputs are not refreshed, so the state this leaves is
    # overwritten by the full timed run below); in eager mode the event-bracketed updates.
    kernel_ms = timed(lambda s: graph.replay(views=False), start, steps)[0] if graph is not None else None
    best, upd_ms = timed(run_step, start, steps)
    if graph is None and wl.refill is None:
        # the whole steps again without the per-call events (their recording costs host time)
        best = timed(lambda s: run_step(s), start, steps)[0]
    errors = [p.errors() for p in pools]
    if any(errors):
        raise SystemExit(f"device error bits set: {errors}")
    if kernel_ms is None:
        kernel_ms = upd_ms
    decode_ms = upd_ms if wl.refill is not None else best  # C5: the updates alone

    total_bytes = sum(wl.step_bytes[start:start + steps])
    gbs = total_bytes / (decode_ms / 1e3) / 1e9
    launches = steps * L
    avg_launch_us = kernel_ms * 1e3 / launches
    bytes_per_launch = total_bytes / launches
    achieved = bytes_per_launch / (avg_launch_us * 1e-6) / 1e9

    traffic, traffic_measured = None, None
    tpath = os.path.join(ROOT, "profiles", f"stream_kernel_c{args.config}_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            windows = json.load(f)["windows"]
        windows = [w for w in windows if w.get("batch") == B]  # this configuration's row count
        for w in windows:
            if w["window_start"] == start and w["steps"] == steps:
                traffic = w["hbm_bytes_per_launch"]
        if traffic is None and windows:
            w = min(windows, key=lambda w: abs(w["algorithmic_bytes_per_launch"] - bytes_per_launch))
            traffic_measured = {"traffic_over_algorithmic": w["traffic_over_algorithmic"],
                                "window_start": w["window_start"], "steps": w["steps"],
                                "context": w["context"]}

    lens = prefill_lengths(cfg)
    kind = cfg["prefill"]
    ctx_lo = min(lens) + start + 1
    workload = (f"{cfg['name']}: {L} layers, batch {B}, {H} KV heads x {D}, {cfg['dtype']}, page {P}; "
                f"prefill ({kind[0]}, context {min(lens)}..{max(lens)}, untimed), then decode steps "
                f"{start}..{start + steps - 1} of the {cfg['decode']}-step trajectory timed (1-token append + "
                f"full contiguous gather per layer; context {ctx_lo}..{max(lens) + start + steps} on the longest "
                f"rows{'; the steps before them run untimed' if start else ''})")
    if "perm_seed" in cfg:
        workload += f"; pages handed out in a seeded random permutation (seed {cfg['perm_seed']})"
    if "occupancy" in cfg:
        workload += (f"; pool of {pools[0].num_pages} pages per layer ({cfg['occupancy']:.0%} occupied after the "
                     f"prefill), {cfg['churn'][0]} seeded rows freed before every step"
                     + (f" and re-prefilled with {lens[0]} tokens (timed apart)" if wl.refill is not None else ""))
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(decode_ms / steps, 4),
        "us_per_step": round(decode_ms * 1e3 / steps, 2),
        "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"].replace("bfloat16", "bf16").replace("float32", "f32").replace("float16", "f16"),
        "data": "synthetic: N(0,1) fp32 rounded to the cache dtype, seeded; inputs resident in HBM",
        "config": {
            "workload": workload,
            "mode": mode + (" + separate commit" if args.separate_commit else ""),
            "layers": L, "batch": B, "kv_heads": H, "head_dim": D, "page_size": P,
            "prefill": kind[0], "decode_steps": steps, "window_start": start, "trajectory_steps": cfg["decode"],
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": KERNEL,
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": int(bytes_per_launch),
            "avg_launch_us": round(avg_launch_us, 3),
        },
    }
    if traffic_measured is not None:
        result["roofline"]["traffic_measured"] = traffic_measured
    if wl.refill is not None:
        refill_ms = best - upd_ms
        result["refill"] = {"rows_per_step": cfg["churn"][0], "tokens_per_row": lens[0],
                            "ms_per_step": round(refill_ms / steps, 3),
                            "gbs": round(wl.refill_bytes * steps / (refill_ms / 1e3) / 1e9, 1),
                            "bytes_per_step": wl.refill_bytes,
                            "step_with_refill_ms": round(best / steps, 3),
                            "note": "free_rows + append_rows of the churned rows, every layer, host-launched"}
    if start > 0:  # the first `steps` steps of the trajectory, for comparison
        first_kernel = timed(lambda s: graph.replay(views=False), 0, steps)[0] if graph is not None else None
        first, first_upd = timed(run_step, 0, steps)
        first_decode = first_upd if wl.refill is not None else first
        fb = sum(wl.step_bytes[:steps])
        fk = first_kernel if first_kernel is not None else first_upd
        result["first_steps"] = {
            "decode_steps": f"0..{steps - 1}", "value": round(fb / (first_decode / 1e3) / 1e9, 2),
            "us_per_step": round(first_decode * 1e3 / steps, 2),
            "avg_launch_us": round(fk * 1e3 / launches, 3), "bytes_per_launch": int(fb / launches),
            "frac": round(fb / launches / (fk * 1e3 / launches * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    if kind[0] == "chunks":
        chunk_bytes = sum(L * (2 * B * kind[2] + 2 * B * (c + 1) * kind[2]) * tok_bytes(cfg) for c in range(kind[1]))
        result["chunked_prefill"] = {"calls_per_layer": kind[1], "seconds_eager": round(prefill_s, 4),
                                     "gbs": round(chunk_bytes / prefill_s / 1e9, 1),
                                     "note": f"{kind[1]} x ({kind[2]}-token append + full gather) per layer, "
                                             f"host-launched, timed with the host clock around the whole phase"}

    if not args.no_cpu_baseline:
        import numpy as np

        from kvgen import to_bits

        cpu_steps = min(cfg["cpu_steps"] or steps, steps)
        layers = 1 if cfg["cpu_steps"] else min(args.cpu_layers or L, L)
        result["cpu_baseline"], want = cpu_baseline(cfg, wl, start, cpu_steps, layers)
        # the GPU's layer 0 after the same steps, from a fresh prefill
        wl.prefill()
        for s in range(start + cpu_steps):
            run_step(s)
        torch.cuda.synchronize()
        if graph is not None:
            seq = wl.pools[0].max_len(B)
            got = (graph.key_out[0][:, :, :seq], graph.value_out[0][:, :, :seq])
        else:
            got = last["out"]
        result["parity"] = {"layer0_kv_bit_exact_vs_cpu_reference": bool(
            np.array_equal(to_bits(got[0]), to_bits(want[0])) and np.array_equal(to_bits(got[1]), to_bits(want[1]))),
            "after_decode_steps": start + cpu_steps}
    if not args.no_attention and cfg["dtype"] in ("bfloat16", "float16") and D == 128:
        attn = attention_leg(cfg, pools, B, dev)
        mid = cfg.get("attention_mid_context")
        if mid and all(int(p.lens[:B].min()) >= mid for p in pools):
            # the trajectory's middle: every row cropped to `mid` positions (the legs after this
            # one prefill again)
            for p in pools:
                p.crop(B, mid)
            m = attention_leg(cfg, pools, B, dev)
            attn["at_mid_context"] = {k: m[k] for k in ("kernel", "context", "us_per_layer_call", "achieved",
                                                       "frac", "bytes_per_call", "parity")}
        result["paged_attention"] = attn
    if args.quant and cfg["dtype"] in ("bfloat16", "float16"):
        result["quantized_kv"] = quant_leg(cfg, wl, steps, dev, decode_ms / steps)
    if not args.no_beam:
        result["beam_select"] = beam_leg(cfg, wl, dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
