#!/usr/bin/env python3
"""Benchmark of the MI355X W4A16 MoE layer (BASELINE.json metric).

Workload (BASELINE.json configs[2] and [3]): one Gemma-4-26B-A4B-shaped MoE
layer -- hidden 2816, 128 experts, top-8 router (bf16 weights ~N(0, 0.02),
fp32 softmax), expert intermediate 704 with fused gate_up [2816 -> 1408] and
down [704 -> 2816], all experts W4A16 at group size 128; activations ~N(0,1).

* decode: M in {1, 8, 32, 64} tokens, uniform routing.  A "step" is one
  layer forward (router + sort + gate_up + gated GELU + down + combine) at
  each M of the sweep.  ``value`` = sum of algorithmic bytes / sum of layer
  times over the sweep (HBM GB/s).  Algorithmic bytes per layer call =
  U * 3,069,440 (packed weights + bf16 scales of the U distinct experts hit)
  + router weights (128 * 2816 * 2) + activations in and out (2 * M * 2816 * 2).
* prefill: M = 4096 tokens, router biased to a Zipf(1.1) expert load with
  empty experts; reported as TFLOP/s over the layer time.
* dense: the W4A16 linear alone (w4a16_linear, quantization.py
  Linear4Bit) at M in {1, 4, 16, 64} x (K, N) in {(2816, 2816), (2816, 1408),
  (704, 2816)}, cycling through enough weight copies that the rotated
  footprint is >= 512 MiB; bytes = N K / 2 + N ceil(K / 128) 2 + M K 2 + M N 2
  per call.  One call is one kernel of 1-4 MB, so these rates include the
  per-launch cost of graph replay.

Weights and inputs are resident in HBM before the timed region; the timed
region replays a HIP graph of layer forwards that cycles through ``--layers``
independent layer copies (default 24 x 393 MB = 9.4 GB; even at M = 1, where
a call touches only its 8 experts, one pass over the copies reads 590 MB,
more than twice the 256 MB Infinity Cache) so every call streams its experts
from HBM.  Times come from HIP events on the stream the kernels run on.

``roofline`` is the dominant decode kernel (the grouped gate_up GEMM at the
largest decode M, about two thirds of the decode bytes), timed alone with each
launch bracketed by its own HIP events (the per-dispatch duration a rocprofv3
kernel trace of the same command reports; the graph-replay mean is recorded
beside it); ``roofline_prefill`` the dominant prefill kernel (the gate_up
stage at M = 4096), timed the same way, against the bf16 MFMA peak, with the
MFMA-busy fraction of the committed counter summary.  ``g32`` repeats decode (M = 1, 64) and prefill at
group size 32, the released checkpoints'.
``cpu_baseline`` times the torch-CPU restatement of the reference's CPU path
(``oracle/torch_cpu.py``) on this host's cores: one decode layer at each M of
the sweep, and configs[0] (the dense W4A16 linear at M = 16).
``ffn_block`` times the whole post-attention FFN block (backends.py:77-126:
norms, shared bf16 MLP, router, experts) per decoder layer at M = 1 and 32.
``bf16_experts`` times the unquantised-experts path (backends.py:209-283) at
M = 1, 8, 64 over 8 rotated copies of a layer's bf16 experts.
``loader`` times checkpoint loading (quantization.py:325-430) of a synthetic
4-layer pack-quantized checkpoint: the reference's host flow against the
device-direct loader.
``latent`` is benchmark configs[4] (30 MoE layers + HybridLink per step, batch
32); ``hybridlink`` times the HybridLink map alone at that batch (weights
rotated through HBM).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from hybridagent_amd import _lib, synth  # noqa: E402

METRIC = "W4A16 MoE layer: decode HBM GB/s (% peak) @M=1..64; prefill TFLOP/s @M=4096"
E, H, I, TOPK, G = 128, 2816, 704, 8, 128
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
EXPERT_BYTES = (2 * I * H // 2 + 2 * I * math.ceil(H / G) * 2) + (H * I // 2 + H * math.ceil(I / G) * 2)
GATEUP_BYTES = 2 * I * H // 2 + 2 * I * math.ceil(H / G) * 2
ROUTER_BYTES = E * H * 2
DECODE_MS = (1, 8, 32, 64)
DENSE_SHAPES = ((2816, 2816), (2816, 1408), (704, 2816))
DENSE_MS = (1, 4, 16, 64)
DENSE_ROTATE_BYTES = 512 * 2 ** 20  # twice the 256 MB Infinity Cache
PREFILL_M = 4096
LATENT_LAYERS, LATENT_BATCH, LATENT_STEPS = 30, 32, 16


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def expert_bytes(g: int) -> int:
    """Packed weights + bf16 scales of one expert (gate_up and down) at group size g."""
    return (2 * I * H // 2 + 2 * I * math.ceil(H / g) * 2) + (H * I // 2 + H * math.ceil(I / g) * 2)


class Layer:
    """One MoE layer's device-resident weights (router + experts)."""

    def __init__(self, seed: int, dev, zipf: bool = False, g: int = G, tiled: bool = True):
        self.g = g
        self.rw = (synth.zipf_router_weights(E, H, seed=seed, device=dev) if zipf
                   else synth.router_weights(E, H, seed=seed, device=dev))
        self.ew = synth.moe_weights(E, H, I, g, seed=seed + 1000, device=dev)
        # load-time tiled copies: the decode streamers' (the decode layers) and
        # the prefill GEMMs' (the Zipf prefill layers); with ``tiled=False`` the
        # kernels read the packed checkpoint layout (the drop-in default)
        ew = self.ew
        self.tiles = _lib.tile_experts(ew.gate_up_packed, ew.gate_up_scale, ew.down_packed, ew.down_scale, g,
                                       decode=not zipf, prefill=zipf) if tiled else None

    def route(self, x):
        rw = self.rw
        return _lib.router_topk(x, rw.scale, rw.scalar_root, rw.proj, rw.per_expert_scale, rw.eps, TOPK)

    def forward(self, x, tiled: bool = True):
        """Router + experts (the MoE half of backends.py:111-122) through one C-ABI call;
        ``tiled=False`` reads the packed checkpoint layout."""
        rw, ew = self.rw, self.ew
        out, _, _ = _lib.moe_layer_forward(x, rw.scale, rw.scalar_root, rw.proj, rw.per_expert_scale,
                                           rw.eps, TOPK, x, ew.gate_up_packed, ew.gate_up_scale,
                                           ew.down_packed, ew.down_scale, group_size=self.g,
                                           tiles=self.tiles if tiled else None)
        return out


def time_graph(fn, calls_per_replay: int, steps: int, warmup: int) -> float:
    """Capture fn() (which issues calls_per_replay layer calls) in a HIP graph and
    return the mean seconds per call over >= steps calls, from HIP events."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    replays = max(1, math.ceil(steps / calls_per_replay))
    for _ in range(max(1, math.ceil(warmup / calls_per_replay))):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e-3 / (replays * calls_per_replay)


def time_dispatches(fns, reps: int, warmup: int = 1) -> float:
    """Mean seconds per launch with each launch bracketed by its own pair of HIP
    events on the stream the kernels run on (eager, one after the other): the
    per-dispatch duration a kernel trace reports, which includes each
    dispatch's completion and so reads slightly above the graph-replay mean."""
    for _ in range(warmup):
        for f in fns:
            f()
    torch.cuda.synchronize()
    pairs = []
    for _ in range(reps):
        for f in fns:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            f()
            b.record()
            pairs.append((a, b))
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in pairs) * 1e-3 / len(pairs)


def decode_sweep(layers, dev, steps, warmup, ms=DECODE_MS, tiled: bool = True):
    out = {}
    g = layers[0].g
    for M in ms:
        x = synth.activations(M, H, seed=7000 + M, device=dev)
        uniq = []
        for ly in layers:
            _, idx = ly.route(x)
            uniq.append(int(torch.unique(idx).numel()))
        U = sum(uniq) / len(uniq)
        t = time_graph(lambda: [ly.forward(x, tiled) for ly in layers], len(layers), steps, warmup)
        nbytes = U * expert_bytes(g) + ROUTER_BYTES + 2 * M * H * 2
        out[M] = {"us": t * 1e6, "unique_experts": U, "bytes": nbytes, "gbps": nbytes / t / 1e9,
                  "frac_hbm": nbytes / t / 1e9 / PEAK_HBM_GBS,
                  "distinct_bytes_per_replay": len(layers) * U * expert_bytes(g)}
        log(f"decode G={g} M={M}{'' if tiled else ' (packed layout)'}: {t*1e6:.1f} us/layer, U={U:.1f}, "
            f"{out[M]['gbps']:.0f} GB/s")
    return out


def gateup_kernel(layers, dev, M, steps, warmup):
    """Time the grouped gate_up GEMM alone (one kernel per call)."""
    x = synth.activations(M, H, seed=7000 + M, device=dev)
    stages, uniq = [], []
    for ly in layers:
        w, idx = ly.route(x)
        st = _lib.MoEStages(M, TOPK, E, H, I, G, dev)
        st.plan(x, idx)
        stages.append(st)
        uniq.append(int(torch.unique(idx).numel()))
    torch.cuda.synchronize()

    fns = [(lambda ly=ly, st=st: st.gate_up(x, ly.ew.gate_up_packed, ly.ew.gate_up_scale, tiles=ly.tiles))
           for ly, st in zip(layers, stages)]
    tg = time_graph(lambda: [f() for f in fns], len(layers), steps, warmup)
    td = time_dispatches(fns, max(1, steps // len(layers)))
    U = sum(uniq) / len(uniq)
    nbytes = U * GATEUP_BYTES + M * H * 2 + M * TOPK * I * 2
    return {"kernel": "k_decode<gateup, tiled> (moe_gate_up_tiled, exact dequantisation)", "M": M,
            "us": td * 1e6, "us_graph": tg * 1e6, "bytes": nbytes, "gbps": nbytes / td / 1e9}


def dense_sweep(dev, steps, warmup):
    """w4a16_linear over rotated weight copies (>= 512 MiB per shape)."""
    out = {}
    for si, (K, N) in enumerate(DENSE_SHAPES):
        wbytes = N * K // 2 + N * math.ceil(K / G) * 2
        nrot = math.ceil(DENSE_ROTATE_BYTES / wbytes)
        packed = synth.packed_int4((nrot, N, K), seed=3000 + si, device=dev)
        scales = synth.group_scales((nrot, N, K), G, seed=3100 + si, device=dev)
        for M in DENSE_MS:
            x = synth.activations(M, K, seed=3200 + M, device=dev)
            t = time_graph(lambda: [_lib.linear(x, packed[i], scales[i], group_size=G) for i in range(nrot)],
                           nrot, steps, warmup)
            nbytes = wbytes + M * K * 2 + M * N * 2
            out[f"K{K}_N{N}_M{M}"] = {"us": t * 1e6, "bytes": nbytes, "gbps": nbytes / t / 1e9,
                                      "frac_hbm": nbytes / t / 1e9 / PEAK_HBM_GBS, "copies": nrot}
            log(f"dense K={K} N={N} M={M}: {t*1e6:.2f} us/call, {nbytes / t / 1e9:.0f} GB/s ({nrot} copies)")
        del packed, scales
        torch.cuda.empty_cache()
    return out


def prefill(dev, steps, warmup, n_layers, g: int = G, stages: bool = True, layer: bool = True):
    """the whole layer (router + sort + gate_up + down + combine) at
    M = 4096 with Zipf routing; with ``stages`` also the gate_up stage alone
    (the grouped gate_up GEMM, the dominant kernel); without ``layer`` only
    that stage (a kernel trace then holds the stage's dispatches alone)."""
    layers = [Layer(seed=9000 + 17 * i, dev=dev, zipf=True, g=g) for i in range(n_layers)]
    x = synth.zipf_activations(PREFILL_M, H, seed=9999, device=dev)
    _, idx = layers[0].route(x)
    counts = torch.bincount(idx.flatten(), minlength=E).cpu()
    flops = 2.0 * PREFILL_M * TOPK * (H * 2 * I + I * H) + 2.0 * PREFILL_M * H * E
    srt = torch.sort(counts, descending=True).values
    res = {"group_size": g, "gflop": flops / 1e9, "empty_experts": int((counts == 0).sum()),
           "hot_expert_rows": srt[:4].tolist()}
    if layer:
        t = time_graph(lambda: [ly.forward(x) for ly in layers], len(layers), steps, warmup)
        res.update({"ms": t * 1e3, "tflops": flops / t / 1e12, "frac_mfma": flops / t / 1e12 / PEAK_BF16_TFLOPS})
        log(f"prefill G={g} M={PREFILL_M}: {t*1e3:.3f} ms/layer, {res['tflops']:.1f} TFLOP/s, "
            f"empty={res['empty_experts']} hot={res['hot_expert_rows']}")
    if stages:
        sts = []
        for ly in layers:
            _, li = ly.route(x)
            st = _lib.MoEStages(PREFILL_M, TOPK, E, H, I, g, dev)
            st.plan(x, li)
            sts.append(st)
        torch.cuda.synchronize()

        fns = [(lambda ly=ly, st=st: st.gate_up(x, ly.ew.gate_up_packed, ly.ew.gate_up_scale, tiles=ly.tiles))
               for ly, st in zip(layers, sts)]
        tg = time_graph(lambda: [f() for f in fns], len(layers), steps, warmup)
        td = time_dispatches(fns, max(1, steps // len(layers)))
        gflop = 2.0 * PREFILL_M * TOPK * H * 2 * I
        res["gate_up_stage"] = {"us": td * 1e6, "us_graph": tg * 1e6, "tflops": gflop / td / 1e12,
                                "gflop": gflop / 1e9}
        log(f"prefill G={g} gate_up stage: {td*1e6:.1f} us per dispatch ({tg*1e6:.1f} us graph-replayed), "
            f"{gflop / td / 1e12:.1f} TFLOP/s")
        del sts
    del layers
    torch.cuda.empty_cache()
    return res


PREFILL_COUNTERS_FILE = os.path.join(ROOT, "profiles", "prefill_M4096_counters.md")


def counter_summary(path, key):
    """A ``key: value`` line of a committed counter summary (None if absent)."""
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith(key + ":"):
                    return float(ln.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def roofline_prefill(pre):
    """The prefill's dominant kernel against the bf16 MFMA peak: the gate_up
    stage (one launch of k_prefill_x<gateup>, the exact-form grouped GEMM),
    algorithmic flops 2 * 4096 * 8 * 2816 * 1408 per launch over its HIP-event
    time."""
    st = pre["gate_up_stage"]
    return {
        "bound": "mfma",
        "kernel": "k_prefill_x<gateup> on the tiled weights (moe_gate_up_tiled stage)",
        "M": PREFILL_M,
        "achieved": round(st["tflops"], 2),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(st["tflops"] / PEAK_BF16_TFLOPS, 4),
        "us_per_launch": round(st["us"], 3),
        "us_per_launch_graph_replay": round(st["us_graph"], 3),
        "timing": "per-dispatch HIP events (each launch bracketed), as a kernel trace reports it",
        "algorithmic_gflop_per_launch": round(st["gflop"], 3),
        "mfma_busy_frac_counter": counter_summary(PREFILL_COUNTERS_FILE, "mfma_busy_frac_gate_up"),
        "counter_source": os.path.relpath(PREFILL_COUNTERS_FILE, ROOT),
        # GFLOP / us = PFLOP/s: x 1e3 for TFLOP/s
        **trace_fields(PREFILL_TRACE_FILE, st["gflop"], PEAK_BF16_TFLOPS, 1e3),
    }


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gateup_decode_M64_traffic.md")
# the committed kernel traces of the two roofline kernels: their per-dispatch
# mean durations (``trace_us_per_launch:`` lines), stated beside this run's
# HIP-event figure so each line's frac can be checked against profiles/
ROOF_TRACE_FILE = os.path.join(ROOT, "profiles", "gateup_decode_M64_kernel_stats.md")
PREFILL_TRACE_FILE = os.path.join(ROOT, "profiles", "prefill_M4096_kernel_stats.md")


def trace_fields(path, work, peak, unit_scale):
    """The committed trace's per-dispatch mean and the fraction of peak it gives
    for ``work`` (bytes or flops per launch; unit_scale turns work/us into the
    peak's unit)."""
    us = counter_summary(path, "trace_us_per_launch")
    if us is None or us <= 0:
        return {"trace_us_per_launch": None, "frac_from_trace": None, "trace_source": None}
    return {"trace_us_per_launch": us, "frac_from_trace": round(work / us * unit_scale / peak, 4),
            "trace_source": os.path.relpath(path, ROOT)}


def measured_traffic():
    """HBM bytes per launch of the roofline kernel from the committed counter
    summary (rocprofv3 FETCH_SIZE / WRITE_SIZE runs scaled by the plain-copy
    calibration); None when no summary is present."""
    try:
        with open(TRAFFIC_FILE) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return int(ln.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def roofline(kern):
    return {
        "bound": "hbm",
        "kernel": kern["kernel"],
        "M": kern["M"],
        "achieved": round(kern["gbps"], 2),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(kern["gbps"] / PEAK_HBM_GBS, 4),
        "traffic": measured_traffic(),
        "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT),
        "us_per_launch": round(kern["us"], 3),
        "us_per_launch_graph_replay": round(kern["us_graph"], 3),
        "timing": "per-dispatch HIP events (each launch bracketed), as a kernel trace reports it",
        "algorithmic_bytes_per_launch": int(kern["bytes"]),
        # B / us = MB/s: / 1e3 for GB/s
        **trace_fields(ROOF_TRACE_FILE, kern["bytes"], PEAK_HBM_GBS, 1e-3),
    }


def calibrate_copy(dev) -> int:
    """A plain device-to-device copy of a known size: what FETCH_SIZE and
    WRITE_SIZE read for it gives the counters' scale on this GPU."""
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(8):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read": n, "bytes_written": n, "calls": 8}))
    return 0


def hybridlink_leg(dev, steps: int = 64):
    """The HybridLink map alone (hybridlink.py:17-28) at the latent loop's
    batch: LayerNorm, proj1 + GELU, proj2 + residual, LayerNorm through
    w4a16_hybridlink.  Ten parameter sets (317 MB) are rotated so the weights
    come from HBM, not the 256 MB last-level cache."""
    from hybridagent_amd.latent import LatentStack
    sets = [LatentStack(0, E, H, I, TOPK, G, seed=8800 + i, device=dev) for i in range(10)]
    x = synth.activations(LATENT_BATCH, H, seed=8899, device=dev)
    t = time_graph(lambda: [st.hybridlink(x) for st in sets], len(sets), steps, 8)
    nbytes = 2 * H * H * 2 + 6 * H * 2 + 2 * LATENT_BATCH * H * 2
    res = {"us": t * 1e6, "batch": LATENT_BATCH, "bytes": nbytes, "gbps": nbytes / t / 1e9,
           "frac_hbm": nbytes / t / 1e9 / PEAK_HBM_GBS}
    log(f"hybridlink B={LATENT_BATCH}: {t*1e6:.2f} us/call, {res['gbps']:.0f} GB/s")
    del sets
    torch.cuda.empty_cache()
    return res


def latent(dev, steps: int = LATENT_STEPS):
    """benchmark configs[4]: 30 MoE layers (h += MoE(RMSNorm(h))) + HybridLink x sqrt(H),
    batch 32, the output fed back as the next step's input.  One HIP graph
    replay = one latent step."""
    from hybridagent_amd.latent import LatentStack
    st = LatentStack(LATENT_LAYERS, E, H, I, TOPK, G, seed=7777, device=dev)
    h0 = synth.activations(LATENT_BATCH, H, seed=7778, device=dev)
    uniq, h = [], h0.clone()
    for i in range(LATENT_LAYERS):  # distinct experts per layer on the first step
        h, idx, _ = st.layer(h, i)
        uniq.append(int(torch.unique(idx).numel()))
    buf = h0.clone()

    def run():
        buf.copy_(st.step(buf))

    t = time_graph(run, 1, steps, 4)
    nbytes = sum(uniq) * EXPERT_BYTES + LATENT_LAYERS * ROUTER_BYTES + 2 * H * H * 2
    res = {"ms_per_step": t * 1e3, "us_per_token": t * 1e6 / LATENT_BATCH, "layers": LATENT_LAYERS,
           "batch": LATENT_BATCH, "steps": steps, "unique_experts_per_layer": sum(uniq) / len(uniq),
           "bytes_per_step": nbytes, "gbps": nbytes / t / 1e9, "frac_hbm": nbytes / t / 1e9 / PEAK_HBM_GBS}
    log(f"latent stack: {t*1e3:.3f} ms/step ({LATENT_LAYERS} layers + HybridLink, batch {LATENT_BATCH}), "
        f"{res['us_per_token']:.1f} us/token, {res['gbps']:.0f} GB/s")
    del st
    torch.cuda.empty_cache()
    return res


def _host_cores() -> int:
    n = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        n = min(n, int(os.environ["OMP_NUM_THREADS"]))
    return max(1, n)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _median_time(fn, budget_s: float, min_reps: int = 3, max_reps: int = 10) -> tuple[float, int]:
    fn()  # warm-up
    times, t_all = [], time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - t_all < budget_s and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all > 3 * budget_s:
            break
    return sorted(times)[len(times) // 2], len(times)


def cpu_baseline(budget_s: float):
    """The reference's CPU path (oracle/torch_cpu.py: the torch ops of
    quantization.py:132-137,171-175,241-294 and the router of backends.py:111-117)
    on this host's cores: one decode layer (router + experts) at each M of the
    decode sweep, value = sum of algorithmic bytes / sum of times as for the
    GPU; and configs[0], Linear4Bit.forward at M = 16, K = N = 2816, G = 128."""
    from oracle import torch_cpu
    ncores = _host_cores()
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(ncores)
    try:
        ew = synth.moe_weights(E, H, I, G, seed=5242)
        rw = synth.router_weights(E, H, seed=4242)
        per_m, tot_b, tot_t, reps = {}, 0.0, 0.0, []
        for M in DECODE_MS:
            x = synth.activations(M, H, seed=7000 + M)

            def layer():
                w, idx, _ = torch_cpu.router(x, rw.scale, rw.scalar_root, rw.proj, rw.per_expert_scale, rw.eps,
                                             TOPK)
                torch_cpu.experts(x, idx, w, ew.gate_up_packed, ew.gate_up_scale, ew.down_packed,
                                  ew.down_scale, G)
                return idx

            U = int(torch.unique(layer()).numel())
            t, n = _median_time(layer, budget_s / len(DECODE_MS))
            nbytes = U * EXPERT_BYTES + ROUTER_BYTES + 2 * M * H * 2
            per_m[str(M)] = {"ms": t * 1e3, "gbps": nbytes / t / 1e9, "unique_experts": U, "reps": n}
            tot_b += nbytes
            tot_t += t
            reps.append(n)
            log(f"cpu baseline decode M={M}: {t*1e3:.1f} ms/layer, {nbytes / t / 1e9:.2f} GB/s ({ncores} threads)")
        # the dense W4A16 linear on the reference CPU path
        x0 = synth.activations(16, 2816, seed=11)
        p0 = synth.packed_int4((2816, 2816), seed=12)
        s0 = synth.group_scales((2816, 2816), G, seed=13)
        t0, n0 = _median_time(lambda: torch_cpu.linear4bit(x0, p0, s0, G), 2.0)
        b0 = 2816 * 2816 // 2 + 2816 * 22 * 2 + 16 * 2816 * 2 * 2
        f0 = 2.0 * 16 * 2816 * 2816
        log(f"cpu baseline configs[0] dense M=16: {t0*1e3:.2f} ms, {f0 / t0 / 1e9:.1f} GFLOP/s")
    finally:
        torch.set_num_threads(prev_threads)
    return {"value": tot_b / tot_t / 1e9, "unit": "GB/s", "cores": ncores, "kind": "port",
            "sample": (f"torch-CPU restatement of the reference CPU path (oracle/torch_cpu.py: router, "
                       f"quantization.py T==1 path at M=1 and the per-expert loop at M>1), one decode layer "
                       f"at each M in {list(DECODE_MS)} (median of {min(reps)}-{max(reps)} reps each), "
                       f"torch {torch.__version__} with {ncores} threads on {_cpu_model()}"),
            "decode": per_m,
            "config0_dense": {"M": 16, "K": 2816, "N": 2816, "group_size": G, "ms": t0 * 1e3, "reps": n0,
                              "gbps": b0 / t0 / 1e9, "gflops": f0 / t0 / 1e9}}


FFN_IM = 2112  # shared-MLP intermediate size assumed for Gemma-4-26B-A4B (config.json absent)
FFN_MS = (1, 32)


class FfnLayer:
    """One decoder layer's FFN-block weights: norms, shared bf16 MLP, router, experts."""

    def __init__(self, seed: int, dev):
        g = torch.Generator(device=dev).manual_seed(seed)
        nrm = lambda: (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
        lin = lambda o, i: (torch.randn(o, i, generator=g, device=dev) / math.sqrt(i)).to(torch.bfloat16)
        self.moe = Layer(seed, dev)
        rw, ew = self.moe.rw, self.moe.ew
        self.args = dict(post_attn_ln_w=nrm(), pre_ff_ln_w=nrm(), mlp_gate_w=lin(FFN_IM, H),
                         mlp_up_w=lin(FFN_IM, H), mlp_down_w=lin(H, FFN_IM), post_ff_ln1_w=nrm(),
                         router_scale=rw.scale, router_scalar_root=rw.scalar_root, router_proj_w=rw.proj,
                         router_per_expert_scale=rw.per_expert_scale, pre_ff_ln2_w=nrm(),
                         gu_packed=ew.gate_up_packed, gu_scale=ew.gate_up_scale, dn_packed=ew.down_packed,
                         dn_scale=ew.down_scale, post_ff_ln2_w=nrm(), post_ff_ln_w=nrm(),
                         layer_scalar=torch.ones(1, dtype=torch.bfloat16, device=dev), eps=1e-6, top_k=TOPK)

    def forward(self, residual, attn_out):
        return _lib.ffn_block(residual, attn_out, **self.args, group_size=G, tiles=self.moe.tiles)


def ffn_leg(dev, steps, warmup, n_layers):
    """The whole post-attention FFN block (backends.py:77-126) per decoder layer at
    decode sizes, cycling through ``n_layers`` independent layer copies (HBM-cold).
    Bytes per call: shared MLP weights 3 * Im * H * 2, the U routed experts,
    router weights, seven norm weights, residual + attn_out in and the output."""
    layers = [FfnLayer(seed=600 + 13 * i, dev=dev) for i in range(n_layers)]
    torch.cuda.synchronize()
    out = {}
    for M in FFN_MS:
        res = synth.activations(M, H, seed=6100 + M, device=dev)
        att = synth.activations(M, H, seed=6200 + M, device=dev)
        uniq = []
        for ly in layers:
            _, idx = ly.moe.route(res)
            uniq.append(int(torch.unique(idx).numel()))
        U = sum(uniq) / len(uniq)
        t = time_graph(lambda: [ly.forward(res, att) for ly in layers], len(layers), steps, warmup)
        nbytes = (3 * FFN_IM * H * 2 + U * EXPERT_BYTES + ROUTER_BYTES + 7 * H * 2 + 3 * M * H * 2)
        out[str(M)] = {"us": t * 1e6, "unique_experts": U, "bytes": nbytes, "gbps": nbytes / t / 1e9,
                       "frac_hbm": nbytes / t / 1e9 / PEAK_HBM_GBS, "shared_mlp_intermediate": FFN_IM}
        log(f"ffn block M={M}: {t*1e6:.1f} us/layer, U={U:.1f}, {nbytes / t / 1e9:.0f} GB/s")
    del layers
    torch.cuda.empty_cache()
    return out


BF16_MS = (1, 8, 64)
BF16_COPIES = 8  # 8 x 1.52 GB; at M = 1 one pass reads 8 x 8 experts x 11.9 MB = 761 MB


def bf16_experts_leg(dev, steps, warmup):
    """The BF16 experts path (backends.py:209-283) at decode sizes over rotated
    copies of a whole layer's bf16 experts; bytes per call = U distinct
    experts x (2I x H + H x I) x 2 + activations in and out."""
    g = torch.Generator(device=dev).manual_seed(1700)
    copies = [((torch.randn(E, 2 * I, H, generator=g, device=dev) / math.sqrt(H)).to(torch.bfloat16),
               (torch.randn(E, H, I, generator=g, device=dev) / math.sqrt(I)).to(torch.bfloat16))
              for _ in range(BF16_COPIES)]
    rw = synth.router_weights(E, H, seed=1701, device=dev)
    out = {}
    for M in BF16_MS:
        x = synth.activations(M, H, seed=1710 + M, device=dev)
        w, idx = _lib.router_topk(x, rw.scale, rw.scalar_root, rw.proj, rw.per_expert_scale, rw.eps, TOPK)
        U = int(torch.unique(idx).numel())
        t = time_graph(lambda: [_lib.bf16_experts_forward(x, idx, w, gu, dn) for gu, dn in copies],
                       len(copies), steps, warmup)
        nbytes = U * (3 * I * H * 2) + 2 * M * H * 2
        out[str(M)] = {"us": t * 1e6, "unique_experts": U, "bytes": nbytes, "gbps": nbytes / t / 1e9,
                       "frac_hbm": nbytes / t / 1e9 / PEAK_HBM_GBS}
        log(f"bf16 experts M={M}: {t*1e6:.1f} us/call, U={U}, {nbytes / t / 1e9:.0f} GB/s")
    del copies
    torch.cuda.empty_cache()
    return out


LOADER_LAYERS, LOADER_SHARDS = 4, 2


def loader_leg(dev, tmpdir: str | None = None):
    """Checkpoint loading (quantization.py:325-430): a synthetic pack-quantized
    checkpoint of LOADER_LAYERS layers x 128 experts at the Gemma shape (1.57 GB,
    LOADER_SHARDS shards, page-cached after writing) loaded into device-resident
    experts modules by (a) the reference's flow -- safetensors load_file on the
    host, per-layer torch.stack / torch.cat of the experts on the host, copy into
    the device buffers -- and (b) the device-direct loader (one pinned read and
    one host-to-device copy per shard, experts written in place on the device).
    GB/s = checkpoint bytes / wall time; the better of two runs each."""
    import shutil
    import tempfile
    import types as _types

    from safetensors.torch import load_file, save_file

    from hybridagent_amd import loader as ld
    from hybridagent_amd.quantization import Gemma4TextExperts4Bit

    d = tempfile.mkdtemp(prefix="w4a16ckpt_", dir=tmpdir)
    try:
        cfg = _types.SimpleNamespace(num_experts=E, hidden_size=H, moe_intermediate_size=I,
                                     hidden_activation="gelu_pytorch_tanh")
        files, nbytes = [], 0
        per = LOADER_LAYERS // LOADER_SHARDS
        for si in range(LOADER_SHARDS):
            sd = {}
            for ly in range(si * per, (si + 1) * per):
                w = synth.moe_weights(E, H, I, G, seed=8100 + ly)
                for e in range(E):
                    pre = f"model.language_model.layers.{ly}.experts.{e}"
                    parts = {"gate_proj": (w.gate_up_packed[e, :I], w.gate_up_scale[e, :I]),
                             "up_proj": (w.gate_up_packed[e, I:], w.gate_up_scale[e, I:]),
                             "down_proj": (w.down_packed[e], w.down_scale[e])}
                    for proj, (pk, sc) in parts.items():
                        sd[f"{pre}.{proj}.weight_packed"] = pk.contiguous()
                        sd[f"{pre}.{proj}.weight_scale"] = sc.contiguous()
            path = os.path.join(d, f"model-{si:05d}-of-{LOADER_SHARDS:05d}.safetensors")
            save_file(sd, path)
            files.append(path)
            nbytes += sum(t.numel() * t.element_size() for t in sd.values())
            del sd
        mods = [Gemma4TextExperts4Bit(cfg, group_size=G).to(dev) for _ in range(LOADER_LAYERS)]

        def reference_flow():
            for path in files:
                sd = load_file(path, device="cpu")
                layers = sorted({ld.parse_expert_key(k)[0] for k in sd})
                for ly in layers:
                    get = lambda proj, kind: torch.stack(
                        [sd[f"model.language_model.layers.{ly}.experts.{e}.{proj}.{kind}"] for e in range(E)])
                    m = mods[ly]
                    m.gate_up_packed.copy_(torch.cat([get("gate_proj", "weight_packed"),
                                                      get("up_proj", "weight_packed")], dim=1))
                    m.gate_up_scale.copy_(torch.cat([get("gate_proj", "weight_scale"),
                                                     get("up_proj", "weight_scale")], dim=1))
                    m.down_packed.copy_(get("down_proj", "weight_packed"))
                    m.down_scale.copy_(get("down_proj", "weight_scale"))
                del sd

        def device_direct():
            ld.stream_shards(files, ld.ExpertPlacer(mods), {}, dev)

        res = {"layers": LOADER_LAYERS, "shards": LOADER_SHARDS, "checkpoint_bytes": nbytes}
        for name, fn in (("reference_flow", reference_flow), ("device_direct", device_direct)):
            best = float("inf")
            for _ in range(2):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                best = min(best, time.perf_counter() - t0)
            res[name] = {"s": best, "gbps": nbytes / best / 1e9}
            log(f"loader {name}: {best:.3f} s for {nbytes / 1e9:.2f} GB, {nbytes / best / 1e9:.2f} GB/s")
        res["speedup"] = res["reference_flow"]["s"] / res["device_direct"]["s"]
        del mods
        torch.cuda.empty_cache()
        return res
    finally:
        shutil.rmtree(d, ignore_errors=True)


def _rounded(v):
    """Floats rounded to 4 decimals, recursively (None passes through)."""
    if isinstance(v, float):
        return round(v, 4)
    if isinstance(v, dict):
        return {k: _rounded(x) for k, x in v.items()}
    if isinstance(v, list):
        return [_rounded(x) for x in v]
    return v


def g32_leg(dev, args):
    """Group size 32, the released checkpoints' (quantization.py:19): decode at
    M = 1 and 64 over the same rotation of layer copies, and the prefill layer."""
    layers = [Layer(seed=200 + 17 * i, dev=dev, g=32) for i in range(args.layers)]
    torch.cuda.synchronize()
    dec = decode_sweep(layers, dev, args.steps, args.warmup, ms=(1, 64))
    del layers
    torch.cuda.empty_cache()
    pre = None if args.no_prefill else prefill(dev, max(8, args.steps // 4), max(2, args.warmup // 4), 4,
                                               g=32, stages=False)
    return {"group_size": 32, "expert_bytes": expert_bytes(32),
            "decode": {str(M): d for M, d in dec.items()}, "prefill": pre}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # layer calls per M; multiples of the 24 rotated layers each graph replay
    # issues, so exactly K calls are timed after W untimed ones
    ap.add_argument("--steps", type=int, default=480)
    ap.add_argument("--warmup", type=int, default=96)
    ap.add_argument("--layers", type=int, default=24,
                    help="independent decode layer copies cycled per graph (24 x 393 MB: at M = 1 the "
                         "8 experts of each copy add up to 590 MB, above twice the 256 MB Infinity Cache)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--only-roofline", action="store_true",
                    help="time only the roofline kernel (for rocprofv3 counter runs)")
    ap.add_argument("--no-latent", action="store_true", help="skip the 30-layer latent stack (configs[4])")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense W4A16 linear sweep (configs[1])")
    ap.add_argument("--only-dense", action="store_true")
    ap.add_argument("--only-latent", action="store_true")
    ap.add_argument("--only-prefill", action="store_true",
                    help="time only the prefill layer (for rocprofv3 counter runs)")
    ap.add_argument("--only-prefill-stage", action="store_true",
                    help="time only the prefill gate_up stage, the prefill roofline kernel (for its kernel trace)")
    ap.add_argument("--no-ffn", action="store_true", help="skip the FFN-block leg")
    ap.add_argument("--no-bf16", action="store_true", help="skip the BF16-experts leg")
    ap.add_argument("--no-loader", action="store_true", help="skip the checkpoint-loading leg")
    ap.add_argument("--only-loader", action="store_true")
    ap.add_argument("--only-bf16", action="store_true")
    ap.add_argument("--only-ffn", action="store_true")
    ap.add_argument("--no-g32", action="store_true",
                    help="skip the group-size-32 leg (the released checkpoints' group size)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run a plain 256 MiB device copy 8 times (counter calibration) and exit")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build's W4A16 MoE path runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured path); run with --gpus 1",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        return calibrate_copy(dev)
    _lib.load()
    torch.manual_seed(0)
    if args.only_latent:
        print(json.dumps({"latent": latent(dev)}), flush=True)
        return 0
    if args.only_loader:
        print(json.dumps({"loader": _rounded(loader_leg(dev))}), flush=True)
        return 0
    if args.only_bf16:
        print(json.dumps({"bf16_experts": _rounded(bf16_experts_leg(dev, args.steps, args.warmup))}), flush=True)
        return 0
    if args.only_ffn:
        print(json.dumps({"ffn_block": _rounded(ffn_leg(dev, args.steps, args.warmup, args.layers))}), flush=True)
        return 0
    if args.only_dense:
        print(json.dumps({"dense": dense_sweep(dev, args.steps, args.warmup)}), flush=True)
        return 0
    if args.only_prefill_stage:
        pre = prefill(dev, max(8, args.steps // 4), max(2, args.warmup // 4), 4, layer=False)
        print(json.dumps({"roofline_prefill": roofline_prefill(pre)}), flush=True)
        return 0
    if args.only_prefill:
        pre = prefill(dev, max(8, args.steps // 4), max(2, args.warmup // 4), 4)
        print(json.dumps({"prefill": pre, "roofline_prefill": roofline_prefill(pre)}), flush=True)
        return 0

    log(f"building {args.layers} decode layers ({args.layers * (E * EXPERT_BYTES + ROUTER_BYTES) / 1e9:.2f} GB)")
    layers = [Layer(seed=100 + 17 * i, dev=dev) for i in range(args.layers)]
    torch.cuda.synchronize()
    if args.only_roofline:
        kern = gateup_kernel(layers, dev, max(DECODE_MS), args.steps, args.warmup)
        print(json.dumps({"roofline": roofline(kern)}), flush=True)
        return 0
    dec = decode_sweep(layers, dev, args.steps, args.warmup)
    # the same layers on the packed checkpoint layout (no tiled copies): what a
    # caller gets without tile_weights()
    dec_packed = decode_sweep(layers, dev, args.steps, args.warmup, tiled=False)
    kern = gateup_kernel(layers, dev, max(DECODE_MS), args.steps, args.warmup)
    log(f"gate_up kernel M={kern['M']}: {kern['us']:.1f} us per dispatch ({kern['us_graph']:.1f} us graph-replayed), "
        f"{kern['gbps']:.0f} GB/s")
    del layers
    torch.cuda.empty_cache()

    pre = None if args.no_prefill else prefill(dev, max(8, args.steps // 4), max(2, args.warmup // 4), 4)
    g32 = None if args.no_g32 else g32_leg(dev, args)
    ffn = None if args.no_ffn else ffn_leg(dev, args.steps, args.warmup, args.layers)
    bf16 = None if args.no_bf16 else bf16_experts_leg(dev, args.steps, args.warmup)
    ldr = None if args.no_loader else loader_leg(dev)

    lat = None if args.no_latent else latent(dev)
    hl = None if args.no_latent else hybridlink_leg(dev)

    dense = None if args.no_dense else dense_sweep(dev, args.steps, args.warmup)

    total_bytes = sum(d["bytes"] for d in dec.values())
    total_t = sum(d["us"] for d in dec.values()) * 1e-6
    value = total_bytes / total_t / 1e9

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_t * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random int4 weights, bf16 scales ~U(0.005,0.02), activations ~N(0,1))",
        "config": {
            "workload": "Gemma-4-26B-A4B-shaped W4A16 MoE layer (router + experts): decode M=1,8,32,64 "
                        "uniform routing (benchmark configs[2]); prefill M=4096 Zipf(1.1) routing (configs[3])",
            "hidden": H, "experts": E, "top_k": TOPK, "intermediate": I, "group_size": G,
            "layers_rotated": args.layers, "timing": "HIP graph replay, HIP events",
            "weights": "decode legs read load-time tiled copies of the experts (+1x expert HBM, "
                       "Gemma4TextExperts4Bit.tile_weights / load_pack_quantized_backbone(tile=True)); "
                       "decode_packed is the same sweep on the packed checkpoint layout",
        },
        "roofline": roofline(kern),
        "roofline_prefill": None if pre is None else _rounded(roofline_prefill(pre)),
        "decode": {str(M): {k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}
                   for M, d in dec.items()},
        "decode_packed": {"value": round(sum(d["bytes"] for d in dec_packed.values()) /
                                         (sum(d["us"] for d in dec_packed.values()) * 1e-6) / 1e9, 2),
                          **{str(M): {k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}
                             for M, d in dec_packed.items()}},
        "prefill": None if pre is None else {k: (round(v, 4) if isinstance(v, float) else v)
                                             for k, v in pre.items()},
        "latent": None if lat is None else {k: (round(v, 4) if isinstance(v, float) else v)
                                            for k, v in lat.items()},
        "hybridlink": None if hl is None else {k: (round(v, 4) if isinstance(v, float) else v)
                                               for k, v in hl.items()},
        "dense": None if dense is None else {c: {k: (round(v, 4) if isinstance(v, float) else v)
                                                 for k, v in d.items()} for c, d in dense.items()},
        "g32": _rounded(g32),
        "ffn_block": _rounded(ffn),
        "bf16_experts": _rounded(bf16),
        "loader": _rounded(ldr),
        "cpu_baseline": _rounded(cpu),
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
