#!/usr/bin/env python3
"""Benchmark: one routed 384-expert top-6 E8P-2bit MoE layer at batch-1 decode
on one MI355X.

A *step* is one pass of the hot path for one token: the whole layer in one
launch (``keep_moe_layer1``, ``moe_layer(one_launch=True)``: dual top-k
router over 384 logits, gate/up/SwiGLU, down and weighted combine, 256
co-resident blocks passing h through a workspace). Every step uses a fresh
routing (64 pre-drawn logit sets), so the 2.42 GB resident code pool streams
from HBM, not from the 256 MB Infinity Cache. Steps are captured in HIP
graphs (64 per graph) and replayed; inputs are resident in HBM before the
timed region. The same layer as two launches (``keep_moe_layer``: router +
gate/up, then down) and as three (router, gate/up, down on the packed-table
kernels) is timed alongside.

``value`` = code-stream bytes of one layer (37,748,736 B: 18 projections of
2048 x 512 uint16 codes; 37,847,040 B with the fp16 row scales, reported as
``layer_bytes_with_scales``) / time per layer, in GB/s, over exactly K timed
steps (after max(W, 1024) untimed warmup steps: the clocks settle over the
first ~5 ms of layers); 32 more replays of the 64-step graph are each timed on their own,
and the median and minimum per layer over those samples are reported beside it.
``roofline`` covers the layer's one launch (``k_moe_layer1``), timed with HIP
events on the stream it is launched on. ``cpu_baseline`` times the C/OpenMP restatement
of the same layer (``oracle/cpu_ref.c``) on the host.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-extra-configs]
[--config {1,2,3,4,5}]

The default line also carries ``config3_verify`` (8, 16 and 64 tokens through
the same layer, each with its HBM roofline over the distinct experts read) and
``config4_prefill`` (2048 tokens, the grouped GEMMs, with the fp16
matrix-core roofline and the matrix-core busy share from the committed
counter summary), measured on the same expert pool after the headline.

``--config`` other than 2 measures the BASELINE's other configurations, one
JSON line per workload, with the same fields (they are parity-test shapes of
the same path, reported beside the headline, not instead of it):
1 one E8P projection (M=1, K=4096, N=2048) from a 384 MiB pool of them, with
the C restatement on the host (all threads and one) and the numpy
dense-decode oracle; 3 speculative verify, the whole layer for M = 8, 16 and
64 tokens (router + gate/up + SwiGLU + down), GB/s over the distinct experts
read; 4 prefill, 2048 tokens with Zipf(1.1) expert popularity (device route
plan + three MFMA grouped GEMMs + SwiGLU + combine), TFLOP/s and GB/s;
5 the 288-expert top-8 layer (4096/1536) with a 50% resident mask as -inf
router bias and tau = 0.3, decode batch 1 and prefill 512 tokens.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16 matrix-core peak of the MI355X
# the arithmetic of the int8 matrix-core paths (decode layer, few-token tiles): decoded E8P weights x 4 are exact int8; activations are split
# into int8 terms under a power-of-two scale per 256-wide slice
DTYPE_Q8 = ("fp16 activations x E8P-2bit (uint16) codes on the int8 matrix cores: x as 3 int8 terms per "
            "256-wide slice (residual <= 2^-20 of the slice max), SwiGLU output h in bf16 as 2 int8 terms "
            "(residual <= 2^-13 of the slice max; 2^-14 in the one-launch layer), exact int32 MFMA sums, fp32 "
            "scaling, SwiGLU and route combine")
# the prefill grouped GEMMs (configs 4 and 5 prefill): fp16 matrix cores, as the reference's fp16 sorted matmul
DTYPE_F16 = ("fp16 activations (bf16 h times a power of two per row, then fp16) x E8P-2bit (uint16) codes "
             "decoded to exact fp16 on the fp16 matrix cores (v_mfma_f32_32x32x16_f16): exact products, fp32 sums, "
             "fp32 scaling, SwiGLU and route combine")
E, H, I, K_TOP = 384, 4096, 2048, 6
GRAPH_STEPS = 64
N_SETS = 64
N_SAMPLES = 32  # timed graph replays behind the median / min
MIN_WARMUP_STEPS = 1024  # untimed layers before the timed region, whatever --warmup asks (at least)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


LAYER_KERNELS = ("k_moe_layer1",)  # the one launch of a layer (keep_moe_layer1)
TWO_LAUNCH_KERNELS = ("k_moeq_route_gateup", "k_moeq_down")  # keep_moe_layer, timed beside it
PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "moe_layer_config2_counters.md")
PROFILE_C4 = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "grouped_gemm_config4_kernel_trace.md")
PREFILL_KERNELS = ("k_gemm_e8_gateup", "k_gemm_e8_down")  # the two grouped GEMMs of a config-4 layer


def mfma_busy(kernels, profile):
    """Matrix-core busy % of each of `kernels` from the committed counter summary (None if absent)."""
    found = {}
    try:
        with open(profile) as f:
            for line in f:
                m = re.match(r"mfma_busy_pct\[(\w+)\] = ([0-9.]+)", line.strip())
                if m:
                    found[m.group(1)] = float(m.group(2))
    except OSError:
        return None
    return {k: found[k] for k in kernels if k in found} or None


def measured_traffic(kernels, profile=PROFILE):
    """HBM bytes of one launch of each of `kernels`, summed, from the committed rocprofv3 counter
    summary (None if any is absent)."""
    found = {}
    try:
        with open(profile) as f:
            for line in f:
                m = re.match(r"traffic_bytes_per_launch\[(\w+)\] = (\d+)", line.strip())
                if m:
                    found[m.group(1)] = int(m.group(2))
    except OSError:
        return None
    if not all(k in found for k in kernels):
        return None
    return sum(found[k] for k in kernels)


def projection_bytes(n: int, k: int, groups: int = 1) -> int:
    return n * (k // 8) * 2 + n * groups * 2


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--config", type=int, default=2, choices=(1, 2, 3, 4, 5),
                    help="BASELINE configuration to measure (2: the headline decode layer)")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="skip the config-3 (verify) and config-4 (prefill) keys of the default line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy kernel (torch.neg, fp16) 8 times, the known-size "
                         "reference that scales FETCH_SIZE / WRITE_SIZE counter readings to bytes")
    ap.add_argument("--measure", choices=("rht", "install"), default=None,
                    help="time a component beside the path instead: the activation RHT kernel (keep_rht) or "
                         "expert installs from a layer-NN.npz into device slot rows")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the routed expert path runs on a single "
                                   "MI355X here (multi-GPU sharding is a design note, not a measured path); "
                                   "run with --gpus 1"}))
        return 2

    if args.measure:
        return measure_component(args)
    if args.config != 2:
        return other_config(args)

    import torch

    import keep_amd
    from keep_amd import _lib, synth
    from keep_amd.ops import _default_codebook, prepared_table

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    lib = _lib.load()
    stream = torch.cuda.Stream(device=dev)  # capture needs a non-default stream (default priority)
    log(f"bench: allocating config-2 pool ({E} experts x 3 projections) on {torch.cuda.get_device_name(dev)}")
    gate = synth.projection(E, I, H, seed=1, device=dev)
    up = synth.projection(E, I, H, seed=2, device=dev)
    down = synth.projection(E, H, I, seed=3, device=dev)
    table = _default_codebook(16, dev)
    prep = prepared_table(table)
    x = synth.rht_activations(1, H, seed=4, device=dev)
    logits = synth.router_logits(N_SETS, E, seed=5, device=dev).reshape(N_SETS, 1, E).contiguous()
    idx = torch.empty((N_SETS, 1, K_TOP), dtype=torch.int32, device=dev)
    w = torch.empty((N_SETS, 1, K_TOP), dtype=torch.float32, device=dev)
    want = torch.empty_like(idx)
    want_s = torch.empty_like(w)
    admit = torch.empty((N_SETS, 1, K_TOP), dtype=torch.uint8, device=dev)
    h = torch.empty((N_SETS, K_TOP * I), dtype=torch.bfloat16, device=dev)  # SwiGLU output held in bf16
    out = torch.empty((N_SETS, H), dtype=torch.float32, device=dev)  # routed sum in fp32
    idx1, w1, h1, out1 = torch.empty_like(idx), torch.empty_like(w), torch.empty_like(h), torch.empty_like(out)
    idx2, w2, out2 = torch.empty_like(idx), torch.empty_like(w), torch.empty_like(out)
    ws_bytes = int(lib.keep_moe_layer1_workspace_bytes(K_TOP, I))
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)  # h exchange + call counter, zeroed once
    F16, BF16, F32 = _lib.KEEP_F16, _lib.KEEP_BF16, _lib.KEEP_F32

    def router(i):
        _lib.check(lib.keep_router_dual_topk(logits[i].data_ptr(), 1, E, K_TOP, None, None, 0, 1, 1.0,
                                             float("inf"), None, 0, idx[i].data_ptr(), w[i].data_ptr(), want[i].data_ptr(),
                                             want_s[i].data_ptr(), admit[i].data_ptr(), stream.cuda_stream),
                   "router")

    def gateup(i):
        _lib.check(lib.keep_moe_gateup(x.data_ptr(), F16, 1, H, I, idx[i].data_ptr(), w[i].data_ptr(), K_TOP, E,
                                       gate.codes.data_ptr(), gate.scales.data_ptr(), up.codes.data_ptr(),
                                       up.scales.data_ptr(), F16, H, table.data_ptr(), prep.data_ptr(), 0.0,
                                       h[i].data_ptr(), stream.cuda_stream), "gateup")

    def down_(i):
        _lib.check(lib.keep_moe_down(BF16, 1, H, I, idx[i].data_ptr(), w[i].data_ptr(), K_TOP, E,
                                     down.codes.data_ptr(), down.scales.data_ptr(), F16, I, table.data_ptr(),
                                     prep.data_ptr(), h[i].data_ptr(), out[i].data_ptr(), F32, stream.cuda_stream),
                   "down")

    def layer(i):  # the split path: router, then gate/up and down on the packed-table kernels
        router(i)
        gateup(i)
        down_(i)

    def layer_one(i):  # the whole layer in one launch (the headline)
        _lib.check(lib.keep_moe_layer1(logits[i].data_ptr(), None, None, 0, 1, 1.0, float("inf"), None, 0, E, K_TOP,
                                       x.data_ptr(), F16, H, I, gate.codes.data_ptr(), gate.scales.data_ptr(),
                                       up.codes.data_ptr(), up.scales.data_ptr(), down.codes.data_ptr(),
                                       down.scales.data_ptr(), F16, H, I, prep.data_ptr(), 0.0, idx2[i].data_ptr(),
                                       w2[i].data_ptr(), None, None, None, ws.data_ptr(), ws_bytes,
                                       out2[i].data_ptr(), F32, stream.cuda_stream), "moe_layer1")

    def layer_two(i):  # keep_moe_layer: router + gate/up in one launch, down in a second
        _lib.check(lib.keep_moe_layer(logits[i].data_ptr(), None, None, 0, 1, 1.0, float("inf"), None, 0, E, K_TOP,
                                      x.data_ptr(), F16, H, I, gate.codes.data_ptr(), gate.scales.data_ptr(),
                                      up.codes.data_ptr(), up.scales.data_ptr(), down.codes.data_ptr(),
                                      down.scales.data_ptr(), F16, H, I, prep.data_ptr(), 0.0, idx1[i].data_ptr(),
                                      w1[i].data_ptr(), None, None, None, h1[i].data_ptr(), out1[i].data_ptr(), F32,
                                      stream.cuda_stream), "moe_layer")

    if args.copy_calibration:
        copy_calibration(torch, dev)
    torch.cuda.synchronize()
    # eager pass: routes for every set, sanity
    with torch.cuda.stream(stream):
        for i in range(N_SETS):
            layer(i)
            layer_two(i)
            layer_one(i)
    torch.cuda.synchronize()
    if not (torch.isfinite(out.float()).all() and torch.isfinite(out1).all() and torch.isfinite(out2).all()):
        raise RuntimeError("non-finite layer output")
    if not (torch.equal(idx1, idx) and torch.equal(idx2, idx)):
        raise RuntimeError("layer kernel routed differently from the router kernel")
    for name, o in (("two-launch", out1), ("one-launch", out2)):
        rel = ((o - out).abs().max() / out.abs().max()).item()
        if not rel <= 2e-3:
            raise RuntimeError(f"{name} layer differs from the split path: max rel {rel:.3e}")

    def capture(fn, n, offset=0):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for j in range(n):
                fn((offset + j) % N_SETS)
        return g

    def timed_replay(graphs, reps_per_graph=1):
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            t0.record(stream)
            for _ in range(reps_per_graph):
                for g in graphs:
                    g.replay()
            t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1)  # ms

    def timed_samples(graphs):
        """Total ms over the graphs, and ms of each replay (events between replays on the launch stream)."""
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(graphs) + 1)]
        with torch.cuda.stream(stream):
            ev[0].record(stream)
            for i, g in enumerate(graphs):
                g.replay()
                ev[i + 1].record(stream)
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[-1]), [ev[i].elapsed_time(ev[i + 1]) for i in range(len(graphs))]

    # capture graphs inside the torch stream context so our raw calls use the capture stream
    with torch.cuda.stream(stream):
        full = capture(layer_one, GRAPH_STEPS)
        tail_n = args.steps % GRAPH_STEPS
        tail = capture(layer_one, tail_n, GRAPH_STEPS) if tail_n else None
        g_two = capture(layer_two, GRAPH_STEPS)
        g_split = capture(layer, GRAPH_STEPS)
        g_gateup = capture(gateup, GRAPH_STEPS)
        g_down = capture(down_, GRAPH_STEPS)
        g_router = capture(router, GRAPH_STEPS)

    n_full = args.steps // GRAPH_STEPS
    # warmup (untimed): W steps, and at least MIN_WARMUP_STEPS (the GPU's clocks settle over the first
    # ~5 ms of back-to-back layers; before that a layer takes up to 10% longer)
    with torch.cuda.stream(stream):
        for _ in range(math.ceil(max(args.warmup, MIN_WARMUP_STEPS) / GRAPH_STEPS)):
            full.replay()
    torch.cuda.synchronize()
    graphs = [full] * n_full + ([tail] if tail is not None else [])
    ms = timed_replay(graphs)
    ms_per_step = ms / args.steps
    # beside the K timed steps: N_SAMPLES replays of the 64-step graph, each timed on its own
    _, per_graph = timed_samples([full] * N_SAMPLES)
    samples_us = sorted(t * 1e3 / GRAPH_STEPS for t in per_graph)

    layer_bytes = K_TOP * (2 * projection_bytes(I, H) + projection_bytes(H, I))
    code_bytes = K_TOP * 3 * I * (H // 8) * 2
    value = code_bytes / (ms_per_step * 1e-3) / 1e9

    # per-kernel averages (HIP events over graph replays on the launch stream)
    reps = max(2, min(16, args.steps // GRAPH_STEPS))
    split_us = timed_replay([g_split], reps) * 1e3 / (reps * GRAPH_STEPS)
    two_us = timed_replay([g_two], reps) * 1e3 / (reps * GRAPH_STEPS)
    gu_us = timed_replay([g_gateup], reps) * 1e3 / (reps * GRAPH_STEPS)
    dn_us = timed_replay([g_down], reps) * 1e3 / (reps * GRAPH_STEPS)
    rt_us = timed_replay([g_router], reps) * 1e3 / (reps * GRAPH_STEPS)
    gu_bytes = K_TOP * 2 * projection_bytes(I, H)
    dn_bytes = K_TOP * projection_bytes(H, I)
    gu_gbps = gu_bytes / (gu_us * 1e-6) / 1e9
    dn_gbps = dn_bytes / (dn_us * 1e-6) / 1e9
    layer_us = ms_per_step * 1e3
    log(f"bench: layer {layer_us:.2f} us ({value:.0f} GB/s), two-launch layer {two_us:.2f} us | split path "
        f"(packed-table kernels) {split_us:.2f} us: "
        f"router {rt_us:.2f}  gateup {gu_us:.2f} ({gu_gbps:.0f} GB/s)  down {dn_us:.2f} ({dn_gbps:.0f} GB/s)")

    result = {
        "metric": "routed VQ-GEMM HBM GB/s (% of 8 TB/s) + MoE-layer decode tok/s, 384e top-6",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_Q8,
        "data": "synthetic: uniform uint16 codes, fp16 log-normal(0,0.3) row scales, RHT'd N(0,1) fp16 "
                "activations, N(0,1) router logits (64 routing sets)",
        "config": {"workload": "config 2: routed decode MoE layer, batch 1, 384 experts, hidden 4096, "
                               "intermediate 2048, SwiGLU, top-6, E8P-2bit, per-row fp16 scales",
                   "tokens": 1, "experts": E, "top_k": K_TOP, "hidden": H, "intermediate": I,
                   "group_size": "per-row", "graph_steps": GRAPH_STEPS},
        "pct_of_8TBps": round(100.0 * value / HBM_PEAK_GBPS, 2),
        "us_per_layer": round(ms_per_step * 1e3, 3),
        "tok_per_s": round(1.0 / (ms_per_step * 1e-3), 1),
        "layer_code_bytes": code_bytes,
        "layer_bytes_with_scales": layer_bytes,
        "gbps_with_scales": round(layer_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        "samples": {"n": len(samples_us), "steps_each": GRAPH_STEPS,
                    "median_us_per_layer": round(float(np.median(samples_us)), 3) if samples_us else None,
                    "min_us_per_layer": round(samples_us[0], 3) if samples_us else None,
                    "max_us_per_layer": round(samples_us[-1], 3) if samples_us else None},
        "path": "keep_moe_layer1 (moe_layer(one_launch=True)): router, gate/up/SwiGLU, down and combine in one "
                "launch of 256 co-resident blocks; keep_moe_layer (two launches) timed beside it",
        "kernels_us": {"moe_layer1 (one launch)": round(layer_us, 3),
                       "moe_layer (two launches: route_gateup + down)": round(two_us, 3),
                       "split_path_packed_table_total": round(split_us, 3),
                       "router": round(rt_us, 3), "moe_gateup": round(gu_us, 3), "moe_down": round(dn_us, 3)},
        "roofline": {"bound": "hbm", "kernel": " + ".join(LAYER_KERNELS), "achieved": round(value, 2),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(value / HBM_PEAK_GBPS, 4),
                     "bytes_per_launch": code_bytes, "us_per_launch": round(layer_us, 3),
                     "traffic": measured_traffic(LAYER_KERNELS),
                     "traffic_two_launch": measured_traffic(TWO_LAUNCH_KERNELS),
                     "traffic_source": "rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0 (copy-calibrated), "
                                       "profiles/moe_layer_config2_counters.md"},
        "cpu_baseline": None,
    }
    if not args.no_extra_configs:
        result.update(extra_configs(torch, stream, gate, up, down, table))
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch, gate, up, down, x, idx, w, table, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


def extra_configs(torch, stream, gate, up, down, table) -> dict:
    """Configs 3 and 4 on the config-2 pool (the same 384 x 4096 / 2048 experts): speculative verify at
    8, 16 and 64 tokens (the whole layer from the logits; HBM roofline over the distinct experts read)
    and prefill at 2048 tokens (the experts' grouped GEMMs; fp16 matrix-core roofline)."""

    from keep_amd.nn import QuantizedVQSwitchGLU, QuantizedVQSwitchLinear, RoutedVQMoE

    def lin(pj, K, Nn):
        return QuantizedVQSwitchLinear(input_dims=K, output_dims=Nn, num_experts=E, codes=pj.codes, scales=pj.scales,
                                       codebook=table, group_size=K, code_bits=16)

    glu = QuantizedVQSwitchGLU(gate_proj=lin(gate, H, I), up_proj=lin(up, H, I), down_proj=lin(down, I, H))
    moe = RoutedVQMoE(glu, top_k=K_TOP)
    expert_b = 2 * projection_bytes(I, H) + projection_bytes(H, I)
    fpr = 2 * 3 * H * I
    c3 = {}
    for T in (8, 16, 64):
        log(f"bench: config 3, {T} tokens")
        c3[f"T{T}"] = verify_point(torch, stream, moe, E, K_TOP, H, I, T, expert_b, fpr)
    log("bench: config 4, 2048 tokens")
    c4 = prefill_point(torch, stream, moe, E, K_TOP, H, I, 2048, expert_b, fpr)
    log("bench: config 3 " + ", ".join(f"T={v['tokens']} {v['us_per_layer']} us" for v in c3.values())
        + f" | config 4 {c4['us_per_layer']} us, {c4['tflops']} TFLOP/s")
    return {"config3_verify": {"workload": "config 3: speculative verify through the config-2 layer (router + fused "
                                           "gate/up/SwiGLU + down/combine), fresh logits per call",
                               "metric_unit": "GB/s over the distinct experts read", **c3},
            "config4_prefill": c4}


def measure_component(args) -> int:
    """One JSON line per workload: keep_rht over fp16 rows of 4096 (T = 1 and the 2048-token
    prefill), HIP events on the launch stream; or expert installs (the config-2 expert size,
    6.3 MB each) from a layer-NN.npz written to a temporary file, timed from the first submit
    to the last copy event (the file is in the page cache: host memory -> pinned -> HBM)."""

    import tempfile

    import torch

    from keep_amd import loaders, rht, synth

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    s = torch.cuda.current_stream(dev)
    if args.measure == "rht":
        signs = torch.from_numpy(np.where(np.random.default_rng(0).integers(0, 2, H) == 0, -1.0, 1.0)
                                 .astype(np.float32)).to(dev)
        side = torch.cuda.Stream(device=dev)  # capture needs a non-default stream (default priority)
        for T in (1, 2048):
            x = torch.randn(T, H, device=dev).half()
            rht.apply_rht(x, signs)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                for _ in range(64):
                    rht.apply_rht(x, signs)
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 20
            a.record(s)
            for _ in range(reps):
                graph.replay()
            b.record(s)
            b.synchronize()
            us = a.elapsed_time(b) * 1000.0 / (reps * 64)
            nbytes = T * H * 2 * 2
            print(json.dumps({"metric": "activation RHT (keep_rht) HBM GB/s", "value": round(nbytes / us / 1e3, 2),
                              "unit": "GB/s", "us_per_launch": round(us, 3), "rows": T, "n": H,
                              "bytes_per_launch": nbytes, "dtype": "fp16 in/out, fp32 butterflies",
                              "note": "64 launches per HIP graph, graph replays timed with HIP events"}), flush=True)
        return 0
    n_exp = 16
    arrays = {}
    for proj, (rows, k), seed in (("w1", (I, H), 1), ("w3", (I, H), 2), ("w2", (H, I), 3)):
        arrays[f"{proj}_codes"], arrays[f"{proj}_scales"] = synth.projection_np(n_exp, rows, k, seed=seed)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "layer-00.npz")
        np.savez(path, code_bits=np.asarray(16), **arrays)
        lf = loaders.LayerFile(path)
        pools = {proj: (torch.zeros((n_exp, *arrays[f"{proj}_codes"].shape[1:]), dtype=torch.int16, device=dev),
                        torch.zeros((n_exp, *arrays[f"{proj}_scales"].shape[1:]), dtype=torch.float16, device=dev))
                 for proj in ("w1", "w3", "w2")}
        inst = loaders.ExpertInstaller(lf, pools, dev)
        inst.submit(0, 0).synchronize()  # warm the pinned allocator
        t0 = time.perf_counter()
        evs = [inst.submit(e, e) for e in range(n_exp)]
        for ev in evs:
            ev.synchronize()
        el = time.perf_counter() - t0
        per = sum(a[0].nbytes for a in arrays.values() if a.ndim == 3)
        ok = all(np.array_equal(pools[p][0].cpu().numpy().view(np.uint16), arrays[f"{p}_codes"]) for p in pools)
        lf.close()
    print(json.dumps({"metric": "expert install GB/s (layer-NN.npz -> pinned -> slot rows)",
                      "value": round(per * n_exp / el / 1e9, 3), "unit": "GB/s", "experts": n_exp,
                      "bytes_per_expert": per, "ms_per_expert": round(el * 1e3 / n_exp, 3), "bytes_match": ok,
                      "note": "file in the page cache; 8 reader threads, 1 MiB pieces"}), flush=True)
    return 0


def cpu_baseline(torch, gate, up, down, x, idx, w, table, seconds):
    """C/OpenMP restatement (oracle/cpu_ref.c) of the same layer on the host:
    LUT decode on the fly, fp32 accumulate, over the routings of 4 sets."""

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import cpu

    nproc, threads = host_threads()
    tab = table.cpu().numpy().view(np.uint32)
    xs = x.float().cpu().numpy()
    sets = []
    for i in range(4):
        ids = idx[i, 0].long()
        pick = lambda p: (p.codes[ids].cpu().numpy().view(np.uint16), p.scales[ids].float().cpu().numpy())  # noqa
        sets.append((pick(gate), pick(up), pick(down), np.arange(K_TOP, dtype=np.int32)[None, :],
                     w[i].cpu().numpy()))
    code_bytes = K_TOP * 3 * I * (H // 8) * 2
    res = {}
    for th, budget in ((threads, seconds), (1, seconds)):
        cpu.moe_decode(xs, sets[0][3], sets[0][4], *sets[0][:3], tab, threads=th)  # warm (LUT build)
        times = []
        t0 = time.perf_counter()
        while True:
            s = sets[len(times) % len(sets)]
            a = time.perf_counter()
            cpu.moe_decode(xs, s[3], s[4], s[0], s[1], s[2], tab, threads=th)
            times.append(time.perf_counter() - a)
            el = time.perf_counter() - t0
            if (el >= budget and len(times) >= 20) or len(times) >= 4000 or el >= 3 * budget:
                break
        res[th] = (float(np.median(times)), float(np.min(times)), len(times), el)
    med, mn, n, el = res[threads]
    med1, mn1, n1, el1 = res[1]
    return {"value": round(code_bytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "nproc": nproc,
            "kind": "port", "us_per_layer_median": round(med * 1e6, 1), "us_per_layer_min": round(mn * 1e6, 1),
            "tok_per_s": round(1.0 / med, 2),
            "one_thread": {"us_per_layer_median": round(med1 * 1e6, 1), "us_per_layer_min": round(mn1 * 1e6, 1),
                           "GB/s": round(code_bytes / med1 / 1e9, 3), "samples": n1},
            "sample": f"config-2 decode layers (4 routings of 6 experts, full 4096/2048 shapes) with "
                      f"oracle/cpu_ref.c (LUT decode, fp32 accumulate): {n} layers in {el:.1f} s on {threads} "
                      f"OpenMP threads (host nproc {nproc}, capped at the box's 16-core share), then {n1} layers "
                      f"in {el1:.1f} s on 1 thread; median per layer, GB/s of the code stream"}


def host_threads():
    """(nproc, threads used): the host's usable cores, capped at the GPU box's 16-core CPU share."""

    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return int(nproc), max(1, min(int(nproc), 16))


def _timed_graph(torch, stream, fn, n_sets, reps, warm=1):
    """us per call of fn(i): a HIP graph of GRAPH_STEPS calls over n_sets
    input sets, replayed `reps` times on `stream` between two events."""

    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for i in range(min(n_sets, GRAPH_STEPS)):  # eager pass: allocations, checks
            fn(i)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for j in range(GRAPH_STEPS):
                fn(j % n_sets)
        for _ in range(warm):
            g.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        t0.record(stream)
        for _ in range(reps):
            g.replay()
        t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e3 / (reps * GRAPH_STEPS)


def _timed_eager(torch, stream, fn, n_sets, iters, warm=2):
    """us per call of fn(i), launched eagerly on `stream` (for paths that size
    their work on the host)."""

    with torch.cuda.stream(stream):
        for i in range(warm):
            fn(i % n_sets)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(iters):
            fn(i % n_sets)
        t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e3 / iters


def _line(metric_value, unit, us, workload, extra, dtype, higher=True, roofline=None, cpu=None, data=None):
    r = {"metric": "routed VQ-GEMM HBM GB/s (% of 8 TB/s) + MoE-layer decode tok/s, 384e top-6",
         "value": round(metric_value, 3), "unit": unit, "n_gpus": 1, "steps": None, "warmup": None,
         "ms_per_step": round(us * 1e-3, 6), "higher_is_better": higher, "scaling": "weak", "vs_baseline": None,
         "dtype": dtype, "data": data or "synthetic: uniform uint16 codes, fp16 log-normal(0,0.3) row scales, "
                                        "RHT'd N(0,1) fp16 activations, N(0,1) router logits",
         "config": dict(workload=workload, **extra), "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(r), flush=True)


def copy_calibration(torch, dev) -> None:
    """Eight plain 256 MiB fp16 copies (torch.neg): read 256 MiB, write 256 MiB each."""

    a = torch.ones(128 << 20, dtype=torch.float16, device=dev)
    b = torch.empty_like(a)
    for _ in range(8):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    del a, b


def other_config(args) -> int:
    import torch

    from keep_amd import _lib, ops, synth
    from keep_amd.nn import QuantizedVQSwitchGLU, QuantizedVQSwitchLinear, RoutedVQMoE
    from keep_amd.router import resident_bias

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)
    cfg = args.config
    reps = 4
    if args.copy_calibration:
        copy_calibration(torch, dev)

    if cfg == 1:
        Ep, N, K = 192, 2048, 4096  # 192 distinct projections = 384 MiB, beyond the 256 MB Infinity Cache
        p = synth.projection(Ep, N, K, seed=11, device=dev)
        x = synth.rht_activations(1, K, seed=12, device=dev)
        table = ops._default_codebook(16, dev)
        outs = [None] * Ep
        code_b = N * (K // 8) * 2
        tot_b = code_b + N * 2

        def fn(i):
            outs[i] = ops.vq_qmv(x[0], p.codes[i], p.scales[i], table, in_dim=K, out_dim=N, group_size=K,
                                 code_bits=16)

        us = _timed_graph(torch, stream, fn, Ep, reps)
        gbps = tot_b / (us * 1e-6) / 1e9
        cpu = None
        if not args.no_cpu_baseline:
            cpu = _cpu_projection(torch, p, x, table, args.cpu_seconds)
        _line(gbps, "GB/s", us, "config 1: one E8P projection, M=1, K=4096, N=2048, per-row fp16 scales "
              "(vq_qmv, 192 distinct projections rotated)", {"tokens": 1, "K": K, "N": N}, "fp16 x E8P, fp32 acc",
              roofline={"bound": "hbm", "kernel": "k_vq_matvec", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes_per_launch": tot_b,
                        "us_per_launch": round(us, 3), "traffic": None}, cpu=cpu)
        return 0

    E, H, I, k = (384, 4096, 2048, 6) if cfg in (3, 4) else (288, 4096, 1536, 8)
    log(f"bench: config {cfg}: allocating {E} experts x 3 projections")
    gate = synth.projection(E, I, H, seed=1, device=dev)
    up = synth.projection(E, I, H, seed=2, device=dev)
    down = synth.projection(E, H, I, seed=3, device=dev)
    table = ops._default_codebook(16, dev)

    def lin(pj, K, Nn):
        return QuantizedVQSwitchLinear(input_dims=K, output_dims=Nn, num_experts=E, codes=pj.codes, scales=pj.scales,
                                       codebook=table, group_size=K, code_bits=16)

    tier, hot_rows = None, None
    res_b = 2 * I * (H // 8) + H * (I // 8) + (2 * I + H) * 2  # 8-bit residual codes + fp16 row scales
    if cfg == 5:  # the 3-bit tier: 8-bit E8 residuals on 10% of the experts (29), all of them resident
        from keep_amd.nn import HotTier
        rng = np.random.default_rng(23)
        resident = np.nonzero(synth.resident_mask(E, frac=0.5, seed=21))[0]
        n_hot = E // 10
        hot = rng.choice(resident, n_hot, replace=False)
        hot_rows = np.full(E, 0xFFFFFFFF, np.uint32)
        hot_rows[hot] = np.arange(n_hot, dtype=np.uint32)

        def res(N, K):
            c = torch.randint(0, 256, (n_hot, N, K // 8), dtype=torch.uint8, device=dev)
            sc = (torch.exp(torch.randn((n_hot, N, 1), device=dev) * 0.3) * 0.1).half()
            return c, sc

        tier = HotTier(hot_rows, {"gate": res(I, H), "up": res(I, H), "down": res(H, I)})
        log(f"bench: config 5: hot tier on {n_hot} resident experts")
    glu = QuantizedVQSwitchGLU(gate_proj=lin(gate, H, I), up_proj=lin(up, H, I), down_proj=lin(down, I, H),
                               hot_tier=tier)
    expert_b = 2 * I * (H // 8) * 2 + H * (I // 8) * 2 + (2 * I + H) * 2  # codes + fp16 row scales
    flops_per_route = 2 * 3 * H * I
    mask = synth.resident_mask(E, frac=0.5, seed=21) if cfg == 5 else None
    bias = resident_bias(torch.from_numpy(mask).to(dev)) if cfg == 5 else None
    moe = RoutedVQMoE(glu, top_k=k, bias_served=bias, bias_demand=None if cfg == 5 else bias,
                      tau=0.3 if cfg == 5 else float("inf"))
    sizes = {3: [8, 16, 64], 4: [2048], 5: [1, 512]}[cfg]
    for T in sizes:
        if cfg == 4:
            pt = prefill_point(torch, stream, moe, E, k, H, I, T, expert_b, flops_per_route)
            _line(pt["tflops"], "TFLOP/s", pt["us_per_layer"], pt["workload"],
                  {"tokens": T, "experts": E, "top_k": k, "hidden": H, "intermediate": I,
                   "distinct_experts": pt["distinct_experts"], "hbm_gbps_distinct": pt["hbm_gbps_distinct"],
                   "pct_of_8TBps": pt["pct_of_8TBps"]}, DTYPE_F16, roofline=pt["roofline"])
            continue
        pt = verify_point(torch, stream, moe, E, k, H, I, T, expert_b, flops_per_route, hot_rows=hot_rows,
                          res_b=res_b)
        one = None
        if cfg == 5 and T == 1:  # the same decode layer in one launch (keep_moe_layer1_nested)
            moe.one_launch = True
            one = verify_point(torch, stream, moe, E, k, H, I, T, expert_b, flops_per_route, hot_rows=hot_rows,
                               res_b=res_b)
            moe.one_launch = False
            log(f"bench: config 5 decode, two launches {pt['us_per_layer']} us, one launch {one['us_per_layer']} us")
        name = {3: f"config 3: speculative verify, {T} tokens through the 384-expert top-6 layer "
                   "(router + fused gate/up/SwiGLU + down/combine)",
                5: f"config 5: 288 experts, top-8, 4096/1536, 50% resident (-inf bias), tau 0.3, 3-bit tier "
                   f"(E8P + 8-bit E8 residual) on 29 experts, {'decode batch 1' if T == 1 else f'prefill {T} tokens'}"
                }[cfg]
        extra = {"distinct_hot_experts": pt["distinct_hot_experts"]} if tier else {}
        if one is not None:
            extra["one_launch"] = {"us_per_layer": one["us_per_layer"], "gbps": one["gbps"],
                                   "pct_of_8TBps": one["pct_of_8TBps"],
                                   "path": "keep_moe_layer1_nested (RoutedVQMoE(one_launch=True))"}
        _line(pt["gbps"], "GB/s", pt["us_per_layer"], name,
              {"tokens": T, "experts": E, "top_k": k, "hidden": H, "intermediate": I,
               "distinct_experts": pt["distinct_experts"], **extra, "tok_per_s": pt["tok_per_s"],
               "pct_of_8TBps": pt["pct_of_8TBps"], "tflops": pt["tflops"]},
              DTYPE_Q8 if T <= 64 else DTYPE_F16, roofline=pt["roofline"])
    return 0


def verify_point(torch, stream, moe, E, k, H, I, T, expert_b, flops_per_route, *, hot_rows=None, res_b=0,
                 n_sets=16, reps=4) -> dict:
    """One layer call of `moe` on T tokens (fresh router logits per call, 16 sets): us per layer, and the
    HBM roofline over the bytes of the distinct experts each call reads (codes + row scales, plus the
    residual tier's rows for its hot experts). Graph-replayed up to 64 tokens, eager above."""

    from keep_amd import synth

    x = synth.rht_activations(T, H, seed=30 + T, device=torch.device("cuda", 0))
    logits = synth.router_logits(n_sets * T, E, seed=50 + T, device=x.device).reshape(n_sets, T, E).contiguous()
    with torch.no_grad():
        sets = [np.unique(moe(x, logits[i])[1].idx.cpu().numpy()) for i in range(n_sets)]
    torch.cuda.synchronize()
    distinct = float(np.mean([len(u) for u in sets]))
    distinct_hot = float(np.mean([int((hot_rows[u] != 0xFFFFFFFF).sum()) for u in sets])) if hot_rows is not None \
        else 0.0
    layer_b = distinct * expert_b + distinct_hot * res_b
    outs = []

    def fn(i):
        outs.append(moe(x, logits[i]))  # keep graph outputs alive

    us = _timed_graph(torch, stream, fn, n_sets, reps) if T <= 64 else _timed_eager(torch, stream, fn, n_sets, 8)
    gbps = layer_b / (us * 1e-6) / 1e9
    return {"tokens": T, "us_per_layer": round(us, 2), "tok_per_s": round(T / (us * 1e-6), 1),
            "distinct_experts": distinct, "distinct_hot_experts": distinct_hot, "gbps": round(gbps, 2),
            "pct_of_8TBps": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "tflops": round(T * k * flops_per_route / (us * 1e-6) / 1e12, 2),
            "roofline": {"bound": "hbm", "kernel": "layer", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes_per_layer": int(layer_b),
                         "us_per_layer": round(us, 2), "traffic": None}}


def prefill_point(torch, stream, moe, E, k, H, I, T, expert_b, flops_per_route) -> dict:
    """The experts of one prefill layer on T tokens with Zipf(1.1) routing (4 route sets, eager: the
    plan sizes its work on the host): us per layer, TFLOP/s against the fp16 matrix-core peak, and the
    HBM rate over the distinct experts read."""

    from keep_amd import synth

    dev = torch.device("cuda", 0)
    x = synth.rht_activations(T, H, seed=30 + T, device=dev)
    idx_np = [synth.zipf_routes(T, E, k, s=1.1, seed=40 + i) for i in range(4)]
    idx = [torch.from_numpy(a).to(dev) for a in idx_np]
    gen = torch.Generator(device=dev).manual_seed(7)
    wts = [torch.softmax(torch.randn(T, k, device=dev, generator=gen), -1) for _ in range(4)]
    distinct = float(np.mean([len(np.unique(a)) for a in idx_np]))

    def fn(i):
        return moe.experts(x, idx[i % 4], wts[i % 4])

    us = _timed_eager(torch, stream, fn, 4, 8)
    flops = T * k * flops_per_route
    tf = flops / (us * 1e-6) / 1e12
    gbps = distinct * expert_b / (us * 1e-6) / 1e9
    busy = mfma_busy(PREFILL_KERNELS, PROFILE_C4)
    return {"tokens": T, "us_per_layer": round(us, 1), "tflops": round(tf, 2), "tok_per_s": round(T / (us * 1e-6), 1),
            "distinct_experts": distinct, "hbm_gbps_distinct": round(gbps, 1),
            "pct_of_8TBps": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "workload": f"config 4: prefill, {T} tokens, Zipf(1.1) routing over {E} experts, top-{k} "
                        "(route plan + 3 MFMA grouped GEMMs + SwiGLU + combine)",
            "roofline": {"bound": "mfma", "kernel": "k_gemm_e8 (gate/up + SwiGLU, then down) with k_gq_rowscale "
                                                    "(h), k_route_plan, k_route_combine", "achieved": round(tf, 2),
                         "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                         "flops_per_layer": flops, "us_per_layer": round(us, 1),
                         "mfma_busy_pct": busy,
                         "traffic": measured_traffic(PREFILL_KERNELS, PROFILE_C4),
                         "traffic_source": "rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0 (copy-calibrated) and "
                                           "SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs / (GRBM_GUI_ACTIVE / 8 XCDs), "
                                           "profiles/grouped_gemm_config4_kernel_trace.md"}}


def _cpu_projection(torch, p, x, table, seconds):
    """Config 1 on the host: the C restatement (all threads, then one) and the
    numpy dense-decode oracle (including its 32 MiB materialisation)."""

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import cpu
    from oracle import ops as oops

    nproc, threads = host_threads()
    tab = table.cpu().numpy().view(np.uint32)
    xs = x.float().cpu().numpy()
    codes = [p.codes[i:i + 1].cpu().numpy().view(np.uint16) for i in range(4)]
    scales = [p.scales[i:i + 1].float().cpu().numpy() for i in range(4)]
    rhs = np.zeros((1, 1), dtype=np.int32)
    res = {}
    for th in (threads, 1):
        cpu.routed_matvec(xs, codes[0], scales[0], tab, rhs, group_size=4096, threads=th)
        n, t0 = 0, time.perf_counter()
        while True:
            cpu.routed_matvec(xs, codes[n % 4], scales[n % 4], tab, rhs, group_size=4096, threads=th)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds / 3 or n >= 20000:
                break
        res[th] = (el / n, n, el)
    n, t0 = 0, time.perf_counter()
    while True:
        oops.qmv(xs[0], codes[n % 4][0], scales[n % 4][0], table=tab)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds / 3 or n >= 200:
            break
    npy = el / n
    b = 2048 * 512 * 2 + 2048 * 2
    per, n_all, el_all = res[threads]
    return {"value": round(b / per / 1e9, 3), "unit": "GB/s", "cores": threads, "nproc": nproc, "kind": "port",
            "us_per_projection": round(per * 1e6, 1),
            "one_thread": {"us_per_projection": round(res[1][0] * 1e6, 1), "GB/s": round(b / res[1][0] / 1e9, 3)},
            "numpy_dense_decode_oracle": {"us_per_projection": round(npy * 1e6, 1),
                                          "note": "includes building the 32 MiB dense fp64 matrix"},
            "sample": f"{n_all} projections in {el_all:.1f} s with oracle/cpu_ref.c (LUT decode, fp32 accumulate, "
                      f"OpenMP {threads} threads), then {res[1][1]} with 1 thread"}


if __name__ == "__main__":
    sys.exit(main())
