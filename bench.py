#!/usr/bin/env python3
"""bench.py -- one MoE layer (MoeRoutingTopK -> MoeExpertFFN -> MoeCombine) per step on one MI355X.

Metric: MoE layer us; FFN TFLOPS & HBM GB/s (% peak), at the decode-size workload
T=128, H=2048, E=16, K=2, I=8192 (fp16 I/O, fp32 accumulation) by default.

A step is one pass of the layer over one batch of synthetic input resident in HBM: routing, the expert FFN
(permute + fused gate/up/SwiGLU grouped GEMM + down grouped GEMM with the expert_out scatter) and combine, all
through the C ABI of libmoe_mi355x.so on one stream, with caller-owned buffers allocated once.
W warm-up steps, then five timed passes of K steps each, every pass between torch.cuda.synchronize() calls:
  1. eager: the three C-ABI calls per step, nothing else recorded -> `value` and `ms_per_step`;
  2. graph replay: one layer step captured once in a HIP graph, replayed untimed and then for K steps (y checked
     bit-exact against the eager y first) -> `layer_us_graph_replay`; G layer steps per graph (--graph-layers,
     default 10, as a serving loop captures a whole forward pass of several MoE layers) ->
     `layer_us_graph_replay_g10` per layer (the key names G). The HIP runtime's graph packet capture is off
     (DEBUG_CLR_GRAPH_PACKET_CAPTURE=0 unless the environment sets it; recorded as `graph_packet_capture`): with
     it on (the runtime's default) one layer per graph replayed ~3.5 us slower than the eager launches;
  3. traced: eager again, with HIP events that the library records around each of its launches on the launch
     stream -> per-kernel average durations, from which `roofline` is computed.
  4. fused: the whole layer in one library call, moe_layer (an optional fast path: on the tiled schedule the
     routing kernel also ranks the slots for the FFN's permute, one launch fewer; on the streaming schedule the
     combine runs in the down projection's reduce); ids, weights, expert_out and y checked bit-exact against the
     three-operator layer first, then W untimed steps -> `layer_us_fused`.
     `value` stays the three-operator layer, the drop-in pipeline.
  5. per-step events: the three-operator layer with an event pair around every step ->
     `layer_us_per_step_events` (p10 / p50 / p90).
Then two library kernels over 1 GiB give this box's achievable HBM rates next to the published 8 TB/s the
roofline uses: a whole-line non-temporal streaming read (`hbm_read_gbps`, the access the decode weight stream
uses) and a plain copy (`hbm_copy_gbps`, read + write); and the vendor library's dense fp16 GEMM (hipBLASLt
through torch.matmul, 8192 x 8192 x 8192, A @ B^T) gives its achievable MFMA rate next to the published
2.5 PFLOP/s (`gemm_fp16_tflops_library`); on workloads of at least 64 rows per expert (and on the prefill pass)
its batched GEMM on the expert GEMMs' own shapes, T*K/E rows for every expert, gives the library's time for the
same flops without the gather, SwiGLU, scatter or ragged experts (`library_bmm`). On the decode workload a prefill pass follows (BASELINE.json
configs[2], T=8192 with the same weights): its FFN time and MFMA fraction are `prefill_ffn_us`,
`prefill_ffn_tflops` and `prefill_ffn_mfma_frac` (the north_star's second target), its kernels under `prefill`.
Kernels whose per-launch inputs fit the 256 MB Infinity
Cache (routing and combine at decode) are flagged `cache_resident`: repeated steps read them from it.

The JSON line also carries:
  roofline      the dominant kernel's algorithmic bytes (or flops) per launch / its average event-timed
                duration, against MI355X's published peaks (HBM 8 TB/s, fp16 dense MFMA 2.5 PFLOP/s); `traffic`
                is the measured HBM bytes per launch from rocprofv3 counters when profiles/traffic.json holds
                them for this workload, else null;
  cpu_baseline  the reference's own NaiveMoE (tests/moe_cpu_sim.cpp, built from its source into oracle/_ref),
                single-threaded on this host, on the first tokens of the same inputs, scaled to a whole layer;
                cpu_baseline_tiled is its TiledMoE on the same sample;
  accuracy      this run's y on those tokens against that NaiveMoE output (the reference's thresholds).
"""
from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import pathlib
import platform
import sys
import time

# Read when the HIP runtime starts, so set before torch is imported. By default the runtime pre-records a captured
# graph's kernel packets and submits them together; on MI355X one layer per graph then replayed at 270.8-271.5 us
# against 267.1-268.3 us for the same launches made eagerly, and with it off at 267.3-268.0 us (three runs each).
os.environ.setdefault("DEBUG_CLR_GRAPH_PACKET_CAPTURE", "0")

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
PKG = "implementing-moe-architecture-operators-on-cann-platform_amd"
METRIC = "MoE layer µs; FFN TFLOPS & HBM GB/s (% peak) at T=128,H=2048,E=16,I=8192"
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20  # MI355X Infinity Cache
RIDGE = MFMA_FP16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)


def progress(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kernel_work(cfg, active_experts: int) -> dict:
    """Algorithmic (bytes, flops) per launch of each kernel; the SwiGLU intermediate round trip through the
    workspace is an implementation cost and is not counted."""
    T, H, E, K, I = cfg.T, cfg.H, cfg.E, cfg.K, cfg.I
    S = T * K
    return {
        "moe_routing_topk": (T * H * 2 + H * E * 2 + S * 6, 2 * T * H * E),
        "moe_permute": (S * 4 * 2 + (E + 1) * 4, 0),
        "moe_ffn_gateup_swiglu": (active_experts * 2 * I * H * 2 + T * H * 2, 4 * S * H * I),
        "moe_ffn_down": (active_experts * I * H * 2 + S * H * 2, 2 * S * H * I),
        "moe_combine": (S * H * 2 + S * 2 + T * H * 2, 2 * S * H),
    }


def roofline_for(name: str, bytes_, flops, avg_ms: float, traffic):
    sec = avg_ms * 1e-3
    intensity = flops / bytes_ if bytes_ else 0.0
    if intensity < RIDGE:
        achieved = bytes_ / sec / 1e9
        return {"kernel": name, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "algorithmic_bytes": bytes_,
                "avg_us": round(avg_ms * 1e3, 2)}
    achieved = flops / sec / 1e12
    return {"kernel": name, "bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_FP16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / MFMA_FP16_PEAK_TFLOPS, 4), "traffic": traffic,
            "algorithmic_flops": flops, "avg_us": round(avg_ms * 1e3, 2)}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def library_bmm_us(torch, dev, T: int, H: int, E: int, K: int, I: int) -> dict:
    """The vendor library's batched fp16 GEMM (hipBLASLt through torch.bmm, fp32 accumulation) on the expert GEMMs'
    shapes with T*K/E rows for every expert: gate/up [E, m, H] x [E, H, 2I], down [E, m, I] x [E, I, H]. A dense
    stand-in for the grouped GEMMs without the row gather, SwiGLU, scatter or ragged experts; both operands
    contiguous. Average event time of 20 launches after 10 warm-up launches (the clock ramps over the first)."""
    m = T * K // E
    out = {"rows_per_expert": m}
    for name, kdim, ndim in (("gateup", H, 2 * I), ("down", I, H)):
        a = torch.randn(E, m, kdim, device=dev, dtype=torch.float16)
        b = torch.randn(E, kdim, ndim, device=dev, dtype=torch.float16).contiguous()
        c = torch.empty(E, m, ndim, device=dev, dtype=torch.float16)
        for _ in range(10):
            torch.bmm(a, b, out=c)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            torch.bmm(a, b, out=c)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / 20 * 1e3
        out[f"{name}_us"] = round(us, 2)
        out[f"{name}_mfma_frac"] = round(2 * E * m * kdim * ndim / (us * 1e-6) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4)
        del a, b, c
    return out


def calibrate_copy(ops, torch, args) -> int:
    """Copy a known number of bytes HBM -> HBM (buffers far larger than the 256 MB Infinity Cache would not be
    needed: the destination is written once and the source read once per launch). A counter run over this mode
    gives the factor that turns FETCH_SIZE / WRITE_SIZE readings into bytes."""
    nbytes = args.calibrate_copy << 20
    dev = torch.device("cuda:0")
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    src.fill_(1)
    for _ in range(args.warmup):
        ops.copy_bytes_(dst, src)
    torch.cuda.synchronize()
    with ops.kernel_trace() as kernels:
        for _ in range(args.steps):
            ops.copy_bytes_(dst, src)
        torch.cuda.synchronize()
    name, (launches, total_ms) = next(iter(kernels.items()))
    avg_ms = total_ms / launches
    print(json.dumps({"mode": "copy calibration", "kernel": name, "bytes_read": nbytes, "bytes_written": nbytes,
                      "launches": launches, "avg_us": round(avg_ms * 1e3, 2),
                      "GB/s (read + write)": round(2 * nbytes / (avg_ms * 1e-3) / 1e9, 1)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="decode", help="workload (synth.CONFIGS); the driver uses the default")
    ap.add_argument("--shape", default=None, metavar="T,H,E,K,I",
                    help="another workload of this shape instead of --config (named 'custom')")
    ap.add_argument("--zipf", action="store_true", help="with --shape: Zipf-skewed routing, as the deepseek config")
    ap.add_argument("--seed", type=int, default=44)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the reference CPU timing")
    ap.add_argument("--cpu-target-gflop", type=float, default=30.0,
                    help="size of the CPU baseline sample in GFLOP of expert FFN work")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay timing")
    ap.add_argument("--graph-layers", type=int, default=10, help="layer steps captured in one HIP graph")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the T=8192 prefill pass that the decode workload adds (prefill_* keys)")
    ap.add_argument("--no-copy-rate", action="store_true",
                    help="skip the achievable-rate probes (1 GiB read and copy, library fp16 GEMM)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead of the layer, run moe_copy_bytes over MIB MiB (reference for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (this build has no multi-GPU "
              "path: expert-parallel sharding with an all-to-all on each side of the FFN is designed, not built)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    ops = importlib.import_module(f"{PKG}.ops")
    synth = importlib.import_module(f"{PKG}.synth")
    lib = importlib.import_module(PKG).load_library()
    if args.calibrate_copy:
        return calibrate_copy(ops, torch, args)
    if args.shape:
        cfg = synth.MoeConfig(*(int(v) for v in args.shape.split(",")), zipf=args.zipf, name="custom")
    else:
        cfg = synth.CONFIGS[args.config]
    T, H, E, K, I = cfg.T, cfg.H, cfg.E, cfg.K, cfg.I
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    progress(f"workload {cfg.name}: T={T} H={H} E={E} K={K} I={I}; generating inputs on the GPU")

    x = torch.empty((T, H), dtype=torch.float16, device=dev)
    ops.synth_normal_f16_(x, args.seed, synth.STREAM_X, 1.0)
    wg = torch.from_numpy(synth.gen_w_gate(cfg, args.seed)).to(dev)
    ew = torch.empty((E, 3 * I, H), dtype=torch.float16, device=dev)
    sa, sb, period, split = synth.expert_weight_sigmas(cfg)
    ops.synth_normal_f16_(ew, args.seed, synth.STREAM_EXPERT_WEIGHTS, sa, sb, period, split)
    ids = torch.empty((T, K), dtype=torch.int32, device=dev)
    w = torch.empty((T, K), dtype=torch.float16, device=dev)
    eo = torch.empty((T, K, H), dtype=torch.float16, device=dev)
    y = torch.empty((T, H), dtype=torch.float16, device=dev)
    ws_bytes = ops.workspace_bytes(T, H, E, K, I)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    sp = int(stream.cuda_stream)
    p = {k: t.data_ptr() for k, t in dict(x=x, wg=wg, ew=ew, ids=ids, w=w, eo=eo, y=y, ws=ws).items()}

    def step(s: int = sp) -> None:
        st = lib.moe_routing_topk(p["x"], p["wg"], p["ids"], p["w"], T, H, E, K, s)
        st |= lib.moe_expert_ffn(p["x"], p["ids"], p["w"], p["ew"], p["eo"], p["ws"], ws_bytes, T, H, E, K, I, s)
        st |= lib.moe_combine(p["eo"], p["ids"], p["w"], p["y"], T, H, K, s)
        if st:
            raise RuntimeError(lib.moe_last_error().decode())

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    y_eager = y.clone()
    progress(f"warm-up done ({args.warmup} steps); timing {args.steps} steps")

    def timed(run_step) -> tuple[float, float]:
        """(host-clock ms, event ms) per step over args.steps steps between synchronisations."""
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        for _ in range(args.steps):
            run_step()
        ev1.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        return (t1 - t0) * 1e3 / args.steps, ev0.elapsed_time(ev1) / args.steps

    # 1) the layer as three eager C-ABI calls per step: the headline value
    ms_per_step, gpu_ms_per_step = timed(step)
    progress(f"eager: {ms_per_step * 1e3:.1f} us/step (host clock), {gpu_ms_per_step * 1e3:.1f} us/step (events)")
    # 2) the same three calls captured in a HIP graph and replayed (no memset nodes: the library records kernels
    #    only); every replay recomputes the whole layer, and its y must equal the eager y bit for bit. Consecutive
    #    graph launches are ~9 us apart on the GPU, so the graph holds G layer steps, as a whole forward pass would;
    #    one layer per graph is timed too.
    graph_ms = graph1_ms = None
    if not args.no_graph:
        def graph_of(layers: int) -> "torch.cuda.CUDAGraph":
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(layers):
                    step(int(torch.cuda.current_stream().cuda_stream))
            y.zero_()
            g.replay()
            torch.cuda.synchronize()
            if not torch.equal(y, y_eager):
                raise RuntimeError("graph replay of the layer differs from the eager layer")
            return g

        def replay_ms(g, layers: int) -> float:
            # untimed replays first: after the capture and the synchronisations the shader clock has dropped, and
            # it takes ~15 launches of the prefill GEMMs to ramp back up
            for _ in range(max(1, args.warmup // layers)):
                g.replay()
            reps = max(1, args.steps // layers)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                g.replay()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / (reps * layers)

        G = max(1, args.graph_layers)
        g = graph_of(G)
        graph_ms = replay_ms(g, G)
        del g
        g = graph_of(1)
        graph1_ms = replay_ms(g, 1)
        del g
        progress(f"graph replay: {graph1_ms * 1e3:.1f} us/layer with one layer per graph, "
                 f"{graph_ms * 1e3:.1f} us/layer with {G} (host clock)")
    # 3) per-kernel HIP events recorded by the library on the launch stream: durations for the roofline
    with ops.kernel_trace() as kernels:
        traced_ms, _ = timed(step)
    progress(f"traced: {traced_ms * 1e3:.1f} us/step with an event pair around every launch")
    # 4) the optional fast path: the whole layer in one call (moe_layer); ids, weights, expert_out and y must
    #    equal the three-operator layer's bit for bit
    ws_layer_bytes = ops.layer_workspace_bytes(T, H, E, K, I)
    ws_layer = torch.empty(ws_layer_bytes, dtype=torch.uint8, device=dev)

    def step_fused(s: int = sp) -> None:
        st = lib.moe_layer(p["x"], p["wg"], p["ew"], p["ids"], p["w"], p["eo"], p["y"], ws_layer.data_ptr(),
                           ws_layer_bytes, T, H, E, K, I, s)
        if st:
            raise RuntimeError(lib.moe_last_error().decode())

    eo_eager, ids_eager, w_eager = eo.clone(), ids.clone(), w.clone()
    y.zero_()
    eo.zero_()
    step_fused()
    torch.cuda.synchronize()
    if not (torch.equal(y, y_eager) and torch.equal(eo, eo_eager) and torch.equal(ids, ids_eager)
            and torch.equal(w, w_eager)):
        raise RuntimeError("the fused layer (moe_layer) differs from the three-operator layer")
    for _ in range(args.warmup):  # the check above left the GPU idle: let the clock ramp up again
        step_fused()
    fused_ms, fused_gpu_ms = timed(step_fused)
    progress(f"fused layer (moe_layer): {fused_ms * 1e3:.1f} us/step (host clock), {fused_gpu_ms * 1e3:.1f} us/step (events)")
    # 5) per-step spread of the three-operator layer: an event pair around every step
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for a, b in evs:
        a.record(stream)
        step()
        b.record(stream)
    torch.cuda.synchronize()
    per_step_us = np.array([a.elapsed_time(b) * 1e3 for a, b in evs])
    spread = {q: round(float(np.percentile(per_step_us, p)), 2) for q, p in (("p10", 10), ("p50", 50), ("p90", 90))}
    progress(f"per-step events: p10 {spread['p10']} / p50 {spread['p50']} / p90 {spread['p90']} us")
    # 6) achievable HBM rate on this box: the library's plain copy kernel over 1 GiB (read + write)
    copy_gbps = read_gbps = None
    if not args.no_copy_rate:
        nb = 1 << 30
        src = torch.empty(nb, dtype=torch.uint8, device=dev)
        dst = torch.empty(nb, dtype=torch.uint8, device=dev)
        src.fill_(1)
        ops.copy_bytes_(dst, src)
        with ops.kernel_trace() as ck:
            for _ in range(5):
                ops.copy_bytes_(dst, src)
            torch.cuda.synchronize()
        (_, (nl, tot_ms)), = ck.items()
        copy_gbps = round(2 * nb / (tot_ms / nl * 1e-3) / 1e9, 1)
        del dst
        ops.stream_read_(src)
        with ops.kernel_trace() as rk:
            for _ in range(5):
                ops.stream_read_(src)
            torch.cuda.synchronize()
        (_, (nl, tot_ms)), = rk.items()
        read_gbps = round(nb / (tot_ms / nl * 1e-3) / 1e9, 1)
        del src
        progress(f"1 GiB: copy kernel {copy_gbps} GB/s (read + write), streaming read {read_gbps} GB/s")
    # 7) achievable dense fp16 MFMA rate on this box: the vendor library's GEMM on a large square problem
    gemm_tflops = None
    if not args.no_copy_rate:
        n = 8192
        ga = torch.randn(n, n, device=dev, dtype=torch.float16)
        gb = torch.randn(n, n, device=dev, dtype=torch.float16)
        for _ in range(10):  # the shader clock ramps over the first launches of a dense MFMA kernel
            gc = ga @ gb.t()
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g0.record()
        for _ in range(20):
            gc = ga @ gb.t()
        g1.record()
        torch.cuda.synchronize()
        gemm_tflops = round(2 * n ** 3 / (g0.elapsed_time(g1) / 20 * 1e-3) / 1e12, 1)
        del ga, gb, gc
        progress(f"library fp16 GEMM {n}^3: {gemm_tflops} TFLOP/s")

    ffn_names = ("moe_permute", "moe_permute_scatter", "moe_ffn_gateup_swiglu", "moe_ffn_gateup_fixup", "moe_ffn_down", "moe_ffn_down_fixup",
                 "moe_ffn_down_reduce")
    # 8) the second north_star target on the same box: the expert FFN of the prefill workload (BASELINE.json
    #    T=8192, same H, E, K, I, so the decode weights are reused with a new x), against the fp16 dense
    #    MFMA peak. Routing, FFN and combine run as in the decode steps; per-kernel HIP events give the FFN time.
    prefill = None
    pcfg = synth.CONFIGS["prefill"]
    if not args.no_prefill and cfg.name == "decode" and (pcfg.H, pcfg.E, pcfg.K, pcfg.I) == (H, E, K, I):
        PT = pcfg.T
        px = torch.empty((PT, H), dtype=torch.float16, device=dev)
        ops.synth_normal_f16_(px, args.seed, synth.STREAM_X, 1.0)
        pwg = torch.from_numpy(synth.gen_w_gate(pcfg, args.seed)).to(dev)
        pids = torch.empty((PT, K), dtype=torch.int32, device=dev)
        pw = torch.empty((PT, K), dtype=torch.float16, device=dev)
        peo = torch.empty((PT, K, H), dtype=torch.float16, device=dev)
        py = torch.empty((PT, H), dtype=torch.float16, device=dev)
        pws_bytes = ops.workspace_bytes(PT, H, E, K, I)
        pws = torch.empty(pws_bytes, dtype=torch.uint8, device=dev)

        def pstep() -> None:
            st = lib.moe_routing_topk(px.data_ptr(), pwg.data_ptr(), pids.data_ptr(), pw.data_ptr(), PT, H, E, K, sp)
            st |= lib.moe_expert_ffn(px.data_ptr(), pids.data_ptr(), pw.data_ptr(), p["ew"], peo.data_ptr(),
                                     pws.data_ptr(), pws_bytes, PT, H, E, K, I, sp)
            st |= lib.moe_combine(peo.data_ptr(), pids.data_ptr(), pw.data_ptr(), py.data_ptr(), PT, H, K, sp)
            if st:
                raise RuntimeError(lib.moe_last_error().decode())

        for _ in range(max(args.warmup, 10)):  # the shader clock ramps over the first launches of the GEMMs
            pstep()
        p_ms, _ = timed(pstep)
        with ops.kernel_trace() as pk:
            timed(pstep)
        pavg = {n: t / c for n, (c, t) in pk.items()}
        p_ffn_ms = sum(pavg[n] for n in ffn_names if n in pavg)
        p_flops = 6 * PT * K * H * I
        gu_flops = 4 * PT * K * H * I
        prefill = {
            "workload": f"prefill MoE layer T={PT},H={H},E={E},K={K},I={I}",
            "layer_us": round(p_ms * 1e3, 2),
            "ffn_us": round(p_ffn_ms * 1e3, 2),
            "ffn_tflops": round(p_flops / (p_ffn_ms * 1e-3) / 1e12, 1),
            "ffn_mfma_frac": round(p_flops / (p_ffn_ms * 1e-3) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
            "gateup_us": round(pavg["moe_ffn_gateup_swiglu"] * 1e3, 2),
            "gateup_mfma_frac": round(gu_flops / (pavg["moe_ffn_gateup_swiglu"] * 1e-3) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
            "kernels_us": {n: round(v * 1e3, 2) for n, v in pavg.items()},
        }
        progress(f"prefill T={PT}: layer {prefill['layer_us']} us, FFN {prefill['ffn_us']} us = "
                 f"{prefill['ffn_tflops']} TFLOP/s ({prefill['ffn_mfma_frac'] * 100:.1f}% of fp16 peak)")
        del px, pwg, pids, pw, peo, py, pws
        if not args.no_copy_rate:
            lib_bmm = library_bmm_us(torch, dev, PT, H, E, K, I)
            prefill["library_bmm"] = lib_bmm
            progress(f"prefill shapes through the library's batched GEMM: {lib_bmm}")

    ids_h = ids.cpu().numpy()
    active = int((np.bincount(ids_h.ravel(), minlength=E) > 0).sum())
    work = kernel_work(cfg, active)
    per_kernel = {}
    for name, (launches, total_ms) in kernels.items():
        avg = total_ms / max(1, launches)
        b, f = work.get(name, (0, 0))
        per_kernel[name] = {"launches": launches, "avg_us": round(avg * 1e3, 2),
                            "GB/s": round(b / (avg * 1e-3) / 1e9, 1) if b else None,
                            "TFLOP/s": round(f / (avg * 1e-3) / 1e12, 2) if f else None,
                            # inputs re-read every step that fit the 256 MB Infinity Cache are served from it
                            "cache_resident": bool(b) and b < MALL_BYTES}
    ffn_ms = sum(kernels[n][1] / kernels[n][0] for n in ffn_names if n in kernels)
    ffn_flops = 6 * T * K * H * I
    ffn_bytes = active * 3 * I * H * 2 + T * H * 2 + T * K * H * 2
    dominant = max(kernels, key=lambda n: kernels[n][1])
    traffic = None
    tfile = ROOT / "profiles" / "traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get(cfg.name, {}).get(dominant)
    db, dflops = work[dominant]
    roofline = roofline_for(dominant, db, dflops, kernels[dominant][1] / kernels[dominant][0], traffic)

    cpu_baseline = None
    cpu_baseline_tiled = None
    accuracy = None
    if not args.no_cpu_baseline:
        import oracle

        if oracle.ref_available():
            per_token = K * 6 * H * I
            n_s = int(max(1, min(T, round(args.cpu_target_gflop * 1e9 / per_token))))
            progress(f"cpu baseline: reference NaiveMoE on the first {n_s} of {T} tokens (1 thread)")
            x_s = x[:n_s].float().cpu().numpy()
            wg_h = wg.float().cpu().numpy()
            ew_h = ew.cpu().numpy().astype(np.float32)
            y_ref, ref_ms = oracle.ref_moe_timed(x_s, wg_h, ew_h, K, I)
            y_tiled, tiled_ms = oracle.ref_moe_timed(x_s, wg_h, ew_h, K, I, tiled=True)
            del ew_h
            cpu_baseline_tiled = {"value": round(tiled_ms * 1e3 * T / n_s, 1), "unit": "us", "cores": 1,
                                  "kind": "reference",
                                  "sample": f"TiledMoE (tests/moe_cpu_sim.cpp:315-569) on the same {n_s} tokens; "
                                            f"{tiled_ms:.0f} ms scaled by {T}/{n_s}"}
            m_t = oracle.compare(y_tiled, y_ref)
            progress(f"cpu baseline (tiled) {tiled_ms:.0f} ms; tiled vs naive max_abs {m_t['max_abs']:.2e}")
            cpu_baseline = {"value": round(ref_ms * 1e3 * T / n_s, 1), "unit": "us", "cores": 1, "kind": "reference",
                            "sample": f"NaiveMoE (tests/moe_cpu_sim.cpp:183-306, g++ -O2 -std=c++17) on the first "
                                      f"{n_s} of {T} tokens, all {E} experts' weights; {ref_ms:.0f} ms scaled by "
                                      f"{T}/{n_s} to one layer",
                            "cpu": cpu_model(), "host_cpus": os.cpu_count()}
            m = oracle.compare(y[:n_s].float().cpu().numpy(), y_ref)
            accuracy = {"tokens": n_s, "max_abs": m["max_abs"], "mean_abs": m["mean_abs"], "cos": m["cos"],
                        "pass": bool(m["max_abs"] < 0.05 and m["mean_abs"] < 0.01 and m["cos"] > 0.99)}
            progress(f"cpu baseline {ref_ms:.0f} ms for {n_s} tokens; accuracy {accuracy}")
        else:
            progress("cpu baseline skipped: oracle/_ref was not built (no reference checkout at build time)")

    layer_us = ms_per_step * 1e3
    result = {
        "metric": METRIC,
        "value": round(layer_us, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (counter-based N(0,1) x; N(0,1/H) w_gate, W_gate, W_up; N(0,1/I) W_down)",
        "config": {"workload": f"{cfg.name} MoE layer T={T},H={H},E={E},K={K},I={I}", "tokens": T,
                   "hidden": H, "experts": E, "top_k": K, "intermediate": I, "active_experts": active},
        "layer_us_gpu_events": round(gpu_ms_per_step * 1e3, 2),
        "layer_us_graph_replay": round(graph1_ms * 1e3, 2) if graph1_ms else None,
        "graph_packet_capture": os.environ.get("DEBUG_CLR_GRAPH_PACKET_CAPTURE"),
        f"layer_us_graph_replay_g{max(1, args.graph_layers)}": round(graph_ms * 1e3, 2) if graph_ms else None,
        "layer_us_traced": round(traced_ms * 1e3, 2),
        "layer_us_fused": round(fused_ms * 1e3, 2),
        "layer_us_per_step_events": spread,
        "ffn_us": round(ffn_ms * 1e3, 2),
        "ffn_tflops": round(ffn_flops / (ffn_ms * 1e-3) / 1e12, 2),
        "ffn_hbm_gbps": round(ffn_bytes / (ffn_ms * 1e-3) / 1e9, 1),
        "ffn_hbm_frac": round(ffn_bytes / (ffn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "ffn_mfma_frac": round(ffn_flops / (ffn_ms * 1e-3) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
        "kernels": per_kernel,
        "hbm_copy_gbps": copy_gbps,
        "hbm_read_gbps": read_gbps,
        "gemm_fp16_tflops_library": gemm_tflops,
        "library_bmm": library_bmm_us(torch, dev, T, H, E, K, I) if not args.no_copy_rate and T * K >= 64 * E else None,
        "prefill_ffn_us": prefill["ffn_us"] if prefill else None,
        "prefill_ffn_tflops": prefill["ffn_tflops"] if prefill else None,
        "prefill_ffn_mfma_frac": prefill["ffn_mfma_frac"] if prefill else None,
        "prefill": prefill,
        "roofline": roofline,
        "cpu_baseline": cpu_baseline,
        "cpu_baseline_tiled": cpu_baseline_tiled,
        "accuracy": accuracy,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
