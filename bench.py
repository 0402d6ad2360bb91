#!/usr/bin/env python3
"""Benchmark of the MI355X GDN-2 forward path (one JSON line on stdout).

Headline workload (`value`): chunked prefill of the default layer,
hidden 2048, 16 heads, head_dim 128, expand_v 1, chunk 64, x ~ N(0,1) of
shape [8, 4096, 2048] through seeded random-init weights (the reference's
initialisers, src/module.rs:121-187, drawn by gdn2_param_init).  One step =
one chunked forward of the recurrence core (chunk-intra + chunk-inter
kernels) over all 8 x 16 x 4096 token-heads, inputs already resident in
HBM.  The projected operands (q, k, g, b, v, w) come from the layer's own
project() once, outside the timed region.

Also reported: the whole layer (hipBLASLt Linear layers + kernels) for the
same prefill; B = 64 fused decode (short conv + gates + L2 norm + step +
gated RMSNorm per token), the kernel alone over 256 tokens with 5 rotating
state buffers (335 MB, larger than the 256 MB MALL; the kernel's time does
not depend on the state values) beside a streaming copy of the same bytes,
and the whole layer over a 2048-token
prefill then 256 single-token steps; the other benchmark configurations
(C1 quick-start, C4 GVA + extensions, C5 long context: core per kernel,
C5's segmented inter passes one by one, and the whole layer); a 1 GiB
device-to-device copy as the measured practical HBM roof; and the CPU
oracle on the same prefill workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "burn-gdn2_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "prefill tokens/s + decode tokens/s (H=16,d=128); % of MFMA/HBM roofline"
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--seq", type=int, default=4096)
    ap.add_argument("--decode-batch", type=int, default=64)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--decode-rotate", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--cpu-batch", type=int, default=8)
    ap.add_argument("--cpu-layer-tokens", type=int, default=4096,
                    help="tokens of the one-sequence sample of the full-layer CPU baseline")
    ap.add_argument("--no-layer", action="store_true")
    ap.add_argument("--settle-ms", type=float, default=150.0,
                    help="untimed back-to-back calls of each timed workload before its warm-ups (the card's clock "
                         "reaches its sustained value after 20-40 ms of continuous load)")
    ap.add_argument("--layer-steps", type=int, default=5)
    ap.add_argument("--warmup-timeline", type=int, metavar="STEPS", default=0,
                    help="only: STEPS back-to-back prefill core steps from an idle card, three times with a 1 s "
                         "host pause between, printed as means over blocks of 20 steps (the clock's warm-up)")
    ap.add_argument("--decode-prefill", type=int, default=2048)
    ap.add_argument("--no-backward", action="store_true", help="skip the chunked backward timing")
    ap.add_argument("--train-only", action="store_true",
                    help="time only the layer training step (forward_train with saved activations + backward)")
    ap.add_argument("--train-summary", metavar="KERNEL_TRACE_CSV",
                    help="per-kernel table of the last training step in a rocprofv3 kernel trace of --train-only")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="end with a 1 GiB device-to-device copy (reference kernel for HBM counters)")
    ap.add_argument("--stats-summary", metavar="KERNEL_STATS_CSV",
                    help="host only: print a rocprofv3 --stats kernel table as markdown and exit")
    ap.add_argument("--timed-summary", metavar="KERNEL_TRACE_CSV",
                    help="host only: mean duration of the dispatches inside bench.py's timed regions (chunk-intra, "
                         "chunk-inter, decode) in a rocprofv3 kernel trace of a default run with the same "
                         "--warmup/--steps/--decode-steps")
    ap.add_argument("--backward-summary", metavar="KERNEL_TRACE_CSV",
                    help="host only: per timed section of a default run's rocprofv3 kernel trace that launches the "
                         "chunked backward or the training forward, the mean duration of each chunk and backward "
                         "kernel over the section's dispatches (warm-up and timed)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other benchmark configurations (C1, C4, C5)")
    ap.add_argument("--configs-only", action="store_true",
                    help="time only the other benchmark configurations (C1, C4, C5) and the copy roof")
    ap.add_argument("--config-steps", type=int, default=10, help="timed core steps per other configuration")
    ap.add_argument("--configs-summary", metavar="KERNEL_TRACE_CSV",
                    help="host only: mean duration of the timed core dispatches of each configuration in a "
                         "rocprofv3 kernel trace of --configs-only with the same --warmup/--config-steps")
    ap.add_argument("--mfma-summary", metavar="COUNTER_CSV",
                    help="host only: per kernel, the MFMA operations by data type and the shader clock from a "
                         "rocprofv3 --pmc run with SQ_INSTS_VALU_MFMA_MOPS_F32 SQ_INSTS_VALU_MFMA_MOPS_BF16 "
                         "SQ_INSTS_VALU_MFMA_MOPS_XF32 SQ_BUSY_CYCLES GRBM_GUI_ACTIVE")
    ap.add_argument("--mix-summary", nargs=2, metavar=("COUNTER_CSV_1", "COUNTER_CSV_2"),
                    help="host only: per-wave instruction mix, MFMA busy and waiting share of the timed kernels "
                         "from two rocprofv3 --pmc runs (SQ_WAVES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_INSTS_VALU "
                         "SQ_INSTS_LDS SQ_INSTS_VMEM_RD SQ_INSTS_VMEM_WR SQ_INSTS_MFMA, then "
                         "SQ_VALU_MFMA_BUSY_CYCLES SQ_WAIT_INST_ANY SQ_WAIT_ANY SQ_LDS_BANK_CONFLICT "
                         "SQ_ACTIVE_INST_VMEM SQ_ACTIVE_INST_LDS SQ_INSTS_SALU GRBM_GUI_ACTIVE)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="host only: per-launch HBM bytes from two rocprofv3 --pmc runs (FETCH_SIZE, "
                         "WRITE_SIZE) of this script with --copy-calibration; writes profiles/*_traffic.json")
    return ap.parse_args()


def load_traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc (profiles/*.json), if present."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        return json.load(fh)


_MARK = {}


def mark(torch, settled):
    """A one-workgroup launch of the library's streaming copy that the trace
    summaries use to find the timed dispatches: 4 floats (stream_copy_kernel)
    before a settle loop, 3 floats (tail_copy_kernel alone) after it."""
    import ctypes

    from gdn2_amd import _capi as CA
    from gdn2_amd.ops import _stream

    if "buf" not in _MARK:
        _MARK["buf"] = torch.zeros(8, device="cuda")
    buf = _MARK["buf"]
    n = 3 if settled else 4
    CA.check(CA.lib().gdn2_stream_copy_f32(ctypes.c_void_p(buf[4:].data_ptr()), ctypes.c_void_p(buf.data_ptr()), n, 1,
                                           _stream()))


def settle(torch, fn, ms):
    """Calls fn back to back, untimed, for `ms` of wall time, between two
    marker launches.  After an idle period (setup, host work) the card runs
    the first 20-40 ms of continuous load at a lower clock than it sustains
    afterwards (chunk-inter measured at 1.55-1.85 GHz there, 2.05-2.3 GHz
    after); the warm-up and timed steps that follow see the sustained clock.
    Returns the number of calls."""
    mark(torch, False)
    n = 0
    t_end = time.perf_counter() + ms / 1e3
    while ms > 0:
        fn()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
            if time.perf_counter() >= t_end:
                break
    torch.cuda.synchronize()
    mark(torch, True)
    return n


def warmup_timeline(torch, G, args, dev):
    """The prefill core (B = 8, T = 4096 operands from the layer's project())
    timed step by step from an idle card: what the settle loops skip."""
    import ctypes

    from gdn2_amd import _capi as CA
    from gdn2_amd.ops import _stream, chunk_args

    cfg = G.Gdn2Config(hidden_size=2048, num_heads=16, head_dim=128, expand_v=1.0, mode="chunk", chunk_size=64)
    layer = G.GatedDeltaNet2(cfg, seed=1337)
    B, T, H, K, V = args.batch, args.seq, cfg.num_heads, cfg.head_dim, cfg.v_head
    gen = torch.Generator(device=dev)
    gen.manual_seed(42)
    P = layer.project(torch.randn((B, T, cfg.hidden_size), generator=gen, device=dev, dtype=torch.float32))
    state = torch.zeros((B, H, K, V), device=dev)
    out = torch.empty((B, T, H, V), device=dev).permute(0, 2, 1, 3)
    ops = [P[n] for n in ("q", "k", "v", "g", "b", "w")]
    ws = torch.empty(G.chunk_workspace_bytes(*ops, state, out, K ** -0.5, 64), dtype=torch.uint8, device=dev)
    cargs = chunk_args(*ops, state, out, K ** -0.5, 64, ws)
    L, stream, pa = CA.lib(), _stream(), ctypes.byref(cargs)
    n, res = max(20, args.warmup_timeline), []
    for phase in range(3):
        time.sleep(1.0)
        torch.cuda.synchronize()
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n)]
        for e in ev:
            e[0].record()
            CA.check(L.gdn2_chunk_intra_f32(pa, stream))
            e[1].record()
            CA.check(L.gdn2_chunk_inter_f32(pa, stream))
            e[2].record()
        torch.cuda.synchronize()
        ti = [e[0].elapsed_time(e[1]) * 1e3 for e in ev]
        te = [e[1].elapsed_time(e[2]) * 1e3 for e in ev]
        for lo in range(0, n - n % 20, 20):
            res.append({"after_idle_s": 1.0, "pass": phase, "steps": [lo, lo + 19],
                        "intra_us": sum(ti[lo:lo + 20]) / 20, "inter_us": sum(te[lo:lo + 20]) / 20})
    layer.close()
    return res


def bench_prefill(torch, G, args, dev):
    """The recurrence core on the layer's own operands: q, k, g, b
    [B, H, T, K] and v, w [B, HV, T, V] from GatedDeltaNet2.project, prepared
    once outside the timed region; out [B, T, HV, V] as the layer writes it;
    then the whole layer (forward_train) for comparison."""
    cfg = G.Gdn2Config(hidden_size=2048, num_heads=16, head_dim=128, expand_v=1.0, mode="chunk", chunk_size=64)
    layer = G.GatedDeltaNet2(cfg, seed=1337)
    B, T, H, K, V, C = args.batch, args.seq, cfg.num_heads, cfg.head_dim, cfg.v_head, 64
    gen = torch.Generator(device=dev)
    gen.manual_seed(42)
    x = torch.randn((B, T, cfg.hidden_size), generator=gen, device=dev, dtype=torch.float32)
    P = layer.project(x)  # q, k, g, b [B, H, T, K]; v, w [B, HV, T, V]
    q, k, g, b = (P[n] for n in ("q", "k", "g", "b"))
    v, w = (P[n] for n in ("v", "w"))
    state = torch.zeros((B, H, K, V), device=dev)
    out = torch.empty((B, T, H, V), device=dev).permute(0, 2, 1, 3)
    scale = K ** -0.5
    from gdn2_amd import _capi as CA
    from gdn2_amd.ops import _stream, chunk_args

    need = G.chunk_workspace_bytes(q, k, v, g, b, w, state, out, scale, C)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    cargs = chunk_args(q, k, v, g, b, w, state, out, scale, C, ws)
    import ctypes

    L = CA.lib()
    stream = _stream()
    pa = ctypes.byref(cargs)

    def step():
        CA.check(L.gdn2_chunk_intra_f32(pa, stream))
        CA.check(L.gdn2_chunk_inter_f32(pa, stream))

    settle(torch, step, args.settle_ms)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
            torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for e0, e1, e2 in evs:
        e0.record()
        CA.check(L.gdn2_chunk_intra_f32(pa, stream))
        e1.record()
        CA.check(L.gdn2_chunk_inter_f32(pa, stream))
        e2.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    intra_all = [e0.elapsed_time(e1) for e0, e1, _ in evs]
    inter_all = [e1.elapsed_time(e2) for _, e1, e2 in evs]
    intra_ms, inter_ms = sum(intra_all) / args.steps, sum(inter_all) / args.steps
    ms_per_step = wall * 1e3 / args.steps
    tokens = B * T
    intra_gflop = B * H * T * 2 * C * (3 * K + V) / 1e9
    inter_gflop = B * H * T * (6 * K * V + 2 * C * V) / 1e9
    kernels = {
        "chunk_intra": {"ms": intra_ms, "ms_median": _median(intra_all), "gflop": intra_gflop,
                        "tflops": intra_gflop / intra_ms, "frac_f32_mfma": intra_gflop / intra_ms / PEAK_F32_TFLOPS},
        "chunk_inter": {"ms": inter_ms, "ms_median": _median(inter_all), "gflop": inter_gflop,
                        "tflops": inter_gflop / inter_ms, "frac_f32_mfma": inter_gflop / inter_ms / PEAK_F32_TFLOPS},
    }
    dom = "chunk_intra" if intra_ms >= inter_ms else "chunk_inter"
    # measured HBM bytes exist for the default workload's shape only
    tr = load_traffic(f"{dom}_b8_t4096_traffic.json") if (B, T) == (8, 4096) else None
    roof = {"kernel": dom, "bound": "mfma", "achieved": kernels[dom]["tflops"], "peak": PEAK_F32_TFLOPS,
            "unit": "TFLOP/s", "frac": kernels[dom]["frac_f32_mfma"],
            "traffic": None if tr is None else tr.get("hbm_bytes_per_launch"),
            "per_launch_gflop": kernels[dom]["gflop"]}
    nb = min(args.cpu_batch, B)
    host = {n: t[:nb].contiguous().cpu().numpy() for n, t in (("q", q), ("k", k), ("v", v), ("g", g), ("b", b),
                                                                ("w", w))}
    del q, k, v, g, b, w, ws, P, out, state
    lay = None
    if not args.no_layer:
        lay = time_layer(torch, lambda: layer.forward_train(x), args.layer_steps, tokens, args.settle_ms)
        lay["gemm_tflop"] = sum(layer_gemm_tflop(cfg, tokens))
        lay.update(time_train_steps(torch, G, layer, x, gen, args, recompute=True))
    layer.close()
    return {"tokens": tokens, "ms_per_step": ms_per_step, "value": tokens / (ms_per_step / 1e3),
            "kernels": kernels, "roofline": roof, "host_sample": host, "scale": scale, "layer": lay}


# The other benchmark configurations: (layer config, batch, tokens, dt_bias
# shift, x seed, description).  C3 (B = 64 decode) is bench_decode's.
OTHER_CONFIGS = {
    "C1": (dict(hidden_size=256, num_heads=4, head_dim=64, expand_v=1.0, mode="chunk", chunk_size=64), 1, 1024, 0.0,
           41, "quick-start layer: hidden 256, 4 heads, head_dim 64, chunk 64, short conv, x [1, 1024, 256]"),
    "C4": (dict(hidden_size=2048, num_heads=8, num_v_heads=16, head_dim=128, expand_v=2.0, allow_neg_eigval=True,
                min_decay=0.9, mode="chunk", chunk_size=64), 4, 8192, 0.0, 44,
           "GVA + extensions: hidden 2048, 8 key heads, 16 value heads, K 128, V 256, neg-eig, min_decay 0.9, "
           "x [4, 8192, 2048] (value heads read key head hv / 2)"),
    "C5": (dict(hidden_size=2048, num_heads=16, head_dim=128, expand_v=1.0, mode="chunk", chunk_size=128), 1, 65536,
           4.0, 45, "long context: hidden 2048, 16 heads, K = V = 128, chunk_size 128, dt_bias + 4, "
                    "x [1, 65536, 2048]"),
    "D256": (dict(hidden_size=2048, num_heads=8, head_dim=256, expand_v=1.0, mode="chunk", chunk_size=64), 8, 4096,
             0.0, 46, "head_dim 256: hidden 2048, 8 heads, K = V = 256, chunk 64, x [8, 4096, 2048]"),
    "V96": (dict(hidden_size=256, num_heads=4, head_dim=64, expand_v=1.5, mode="chunk", chunk_size=64), 8, 4096,
            0.0, 47, "the reference's CPU-benchmark layer (tests/bit_exact.rs:224-235): hidden 256, 4 heads, K 64, "
                     "expand_v 1.5 (V 96), x [8, 4096, 256]"),
}
# configurations whose chunked backward is timed too: head_dim 256, V = 96 (two-wave
# reverse-recurrence workgroups) and the long context's strong decays (the exact
# diagonal terms of the decay pass, the segmented reverse recurrence)
BWD_CONFIGS = ("C5", "D256", "V96")
# configurations whose core is also timed on the per-token scan (gdn2_recurrent_fwd_f32,
# the path their head shapes took before the chunk kernels covered them)
SCAN_COMPARE = ("V96",)


def bench_other_config(torch, G, args, dev, name):
    """One of the other benchmark configurations: the recurrence core on the
    layer's own project() operands (chunk-intra, then chunk-inter; with more
    than one segment its three passes timed one by one), then the whole layer
    (forward_train).  The kernels always work on 64-token chunks (the result
    does not depend on the chunk size beyond rounding), so the algorithmic
    work is counted at C = 64."""
    import ctypes

    from gdn2_amd import _capi as CA
    from gdn2_amd.ops import _stream, chunk_args

    over, B, T, dt_shift, xseed, desc = OTHER_CONFIGS[name]
    cfg = G.Gdn2Config(**over)
    layer = G.GatedDeltaNet2(cfg, seed=1337)
    if dt_shift:
        layer.set_param("dt_bias", layer.param("dt_bias") + dt_shift)
    gen = torch.Generator(device=dev)
    gen.manual_seed(xseed)
    x = torch.randn((B, T, cfg.hidden_size), generator=gen, device=dev, dtype=torch.float32)
    P = layer.project(x)
    q, k, g, b, v, w = (P[n] for n in ("q", "k", "g", "b", "v", "w"))
    HV, K, V, C = cfg.hv, cfg.head_dim, cfg.v_head, 64
    state = torch.zeros((B, HV, K, V), device=dev)
    out = torch.empty((B, T, HV, V), device=dev).permute(0, 2, 1, 3)
    scale = K ** -0.5
    need = G.chunk_workspace_bytes(q, k, v, g, b, w, state, out, scale, C)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    cargs = chunk_args(q, k, v, g, b, w, state, out, scale, C, ws)
    L, stream, pa = CA.lib(), _stream(), ctypes.byref(cargs)
    nseg = int(L.gdn2_chunk_segments(pa))
    passes = (1, 2, 3) if nseg > 1 else (3,)

    def step(evs=None):
        if evs:
            evs[0].record()
        CA.check(L.gdn2_chunk_intra_f32(pa, stream))
        for i, ps in enumerate(passes):
            if evs:
                evs[1 + i].record()
            CA.check(L.gdn2_chunk_inter_pass_f32(pa, ps, stream))
        if evs:
            evs[-1].record()

    settle(torch, step, args.settle_ms)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    reps = max(1, args.config_steps)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(passes) + 2)] for _ in range(reps)]
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    intra = [e[0].elapsed_time(e[1]) for e in evs]
    per_pass = [[e[1 + i].elapsed_time(e[2 + i]) for e in evs] for i in range(len(passes))]
    inter = [sum(pp[r] for pp in per_pass) for r in range(reps)]
    intra_ms, inter_ms = sum(intra) / reps, sum(inter) / reps
    tokens = B * T
    intra_gflop = B * HV * T * 2 * C * (3 * K + V) / 1e9
    inter_gflop = B * HV * T * (6 * K * V + 2 * C * V) / 1e9
    core_ms = intra_ms + inter_ms
    res = {"workload": desc, "batch": B, "seq_len": T, "tokens": tokens, "kernel_chunk": C,
           "core": {"ms_per_step": core_ms, "tokens_per_s": tokens / (core_ms / 1e3), "steps": reps,
                    "chunk_intra": {"ms": intra_ms, "ms_median": _median(intra), "gflop": intra_gflop,
                                    "tflops": intra_gflop / intra_ms,
                                    "frac_f32_mfma": intra_gflop / intra_ms / PEAK_F32_TFLOPS},
                    "chunk_inter": {"ms": inter_ms, "ms_median": _median(inter), "gflop": inter_gflop,
                                    "tflops": inter_gflop / inter_ms,
                                    "frac_f32_mfma": inter_gflop / inter_ms / PEAK_F32_TFLOPS,
                                    "segments": nseg}}}
    if nseg > 1:
        names = ("segment_summaries", "chain", "output_pass")
        res["core"]["chunk_inter"]["passes_ms"] = {n: sum(pp) / reps for n, pp in zip(names, per_pass)}
    if name in BWD_CONFIGS and not args.no_backward:
        res["backward"] = time_chunk_backward(torch, args, dev, q, k, g, b, v, w, desc, scan=name in SCAN_COMPARE)
    if name in SCAN_COMPARE:
        from gdn2_amd.ops import _p, _strides3

        ra = CA.RecurrentArgs(_p(q), _p(k), _p(g), _p(b), _p(v), _p(w), _p(state), _p(state), _p(out), B,
                              cfg.num_heads, HV, T, K, V, *_strides3(q), *_strides3(v), *_strides3(out), scale)
        rp = ctypes.byref(ra)
        scan = lambda: CA.check(L.gdn2_recurrent_fwd_f32(rp, stream))
        settle(torch, scan, args.settle_ms)
        scan()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            scan()
        e1.record()
        torch.cuda.synchronize()
        scan_ms = e0.elapsed_time(e1) / reps
        res["core"]["scan"] = {"ms_per_step": scan_ms, "tokens_per_s": tokens / (scan_ms / 1e3),
                               "chunk_speedup": scan_ms / core_ms, "kernel": "gdn2_recurrent_fwd_f32"}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_config_core(name, [t[:1].contiguous().cpu().numpy() for t in (q, k, v, g, b, w)],
                                              scale)
    del P, q, k, g, b, v, w, ws, out, state
    torch.cuda.empty_cache()
    if not args.no_layer:
        lay = time_layer(torch, lambda: layer.forward_train(x), max(1, min(args.layer_steps, 3)), tokens,
                         args.settle_ms)
        lay["gemm_tflop"] = sum(layer_gemm_tflop(cfg, tokens))
        res["layer"] = lay
    del x
    layer.close()
    torch.cuda.empty_cache()
    return res


def bench_copy_roof(torch, dev, reps=10):
    """The practical HBM roof: a 1 GiB device-to-device copy (read + write
    2 GiB per copy), timed with events: the library's streaming copy
    (gdn2_stream_copy_f32) at a few grid sizes, the best kept, and torch's
    copy_ beside it."""
    import ctypes

    from gdn2_amd import _capi as CA
    from gdn2_amd.ops import _stream

    src = torch.ones(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    L, stream = CA.lib(), _stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    per_grid = {}
    for wg in (2048, 4096, 8192, 16384):
        ms = timed(lambda: CA.check(L.gdn2_stream_copy_f32(ctypes.c_void_p(dst.data_ptr()),
                                                            ctypes.c_void_p(src.data_ptr()), src.numel(), wg,
                                                            stream)))
        per_grid[wg] = 2 * COPY_BYTES / (ms / 1e3) / 1e9
    torch_gbs = 2 * COPY_BYTES / (timed(lambda: dst.copy_(src)) / 1e3) / 1e9
    ok = bool(torch.equal(dst, src))
    del src, dst
    torch.cuda.empty_cache()
    wg = max(per_grid, key=per_grid.get)
    gbs = per_grid[wg]
    return {"GBs": gbs, "bytes_moved": 2 * COPY_BYTES, "frac_of_peak": gbs / PEAK_HBM_GBS, "workgroups": wg,
            "GBs_per_grid": per_grid, "torch_copy_GBs": torch_gbs, "copy_ok": ok,
            "what": "1 GiB device-to-device copy (gdn2_stream_copy_f32, best grid), read + write"}


def decode_copy_roof(torch, dev, bytes_step, steps, nrot):
    """The decode step's bytes as a plain copy: gdn2_stream_copy_f32 reading
    and writing bytes_step / 2 each, over nrot rotating buffer pairs like the
    decode's states, best of a few grid sizes.  The decode kernel's time
    against it is its distance from a streaming kernel of the same size."""
    import ctypes

    from gdn2_amd import _capi as CA
    from gdn2_amd.ops import _stream

    n = bytes_step // 8 // 4 * 4
    src = [torch.ones(n, device=dev) for _ in range(nrot)]
    dst = [torch.empty(n, device=dev) for _ in range(nrot)]
    L, stream = CA.lib(), _stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = None
    for wg in (512, 1024, 2048):
        def one(t):
            CA.check(L.gdn2_stream_copy_f32(ctypes.c_void_p(dst[t % nrot].data_ptr()),
                                            ctypes.c_void_p(src[t % nrot].data_ptr()), n, wg, stream))
        for t in range(8):
            one(t)
        torch.cuda.synchronize()
        e0.record()
        for t in range(steps):
            one(t)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / steps * 1e3
        if best is None or us < best["us"]:
            best = {"us": us, "GBs": 8 * n / (us / 1e6) / 1e9, "workgroups": wg}
    del src, dst
    torch.cuda.empty_cache()
    best["bytes"] = 8 * n
    return best


def mfma_summary(path, n_se=32, n_xcc=8):
    """MFMA operations (the MOPS counters count 512 flops each) by data type
    and the clock per kernel, over dispatches longer than 100 us:
    SQ_BUSY_CYCLES summed over the 32 shader engines and GRBM_GUI_ACTIVE
    summed over the 8 XCDs, each divided by the dispatch duration.  hipBLASLt
    kernels are labelled by their macro tile; only the timed shapes' dispatches
    (the longest of each label) are kept, the candidates timed at plan
    creation fall out as slower ones."""
    import collections
    import csv
    import re

    by = collections.defaultdict(dict)
    for r in csv.DictReader(open(path)):
        d = by[int(r["Dispatch_Id"])]
        d["name"] = r["Kernel_Name"]
        d["us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    groups = collections.defaultdict(list)
    for d in by.values():
        if d["us"] < 100:
            continue
        n = d["name"]
        if n.startswith("Cijk"):
            m = re.search(r"MT\d+x\d+x\d+", n)
            label = f"hipBLASLt {n[:18]} {m.group(0) if m else ''}"
        else:
            label = _short(n)
        groups[(label, round(d.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0)))].append(d)
    # per GEMM shape (its flop count), the algorithm the plan kept is the one run most often
    best = {}
    for (label, fl), ds in groups.items():
        if label.startswith("hipBLASLt") and len(ds) > len(groups.get(best.get(fl), [])):
            best[fl] = (label, fl)
    groups = {k: v for k, v in groups.items() if not k[0].startswith("hipBLASLt") or best.get(k[1]) == k}
    print("| kernel | dispatches | mean us | F32 MFMA GFLOP | BF16 | XF32 | F32 TFLOP/s | clock GHz "
          "(SQ_BUSY_CYCLES / 32 SE) | clock GHz (GRBM_GUI_ACTIVE / 8 XCD) |")
    print("|---|---|---|---|---|---|---|---|---|")
    for (label, _), ds in sorted(groups.items(), key=lambda kv: -sum(d["us"] for d in kv[1]))[:16]:
        us = sum(d["us"] for d in ds) / len(ds)
        f32 = sum(d.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0) for d in ds) / len(ds) * 512 / 1e9
        bf = sum(d.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) for d in ds) / len(ds) * 512 / 1e9
        xf = sum(d.get("SQ_INSTS_VALU_MFMA_MOPS_XF32", 0.0) for d in ds) / len(ds) * 512 / 1e9
        sq = sum(d.get("SQ_BUSY_CYCLES", 0.0) for d in ds) / len(ds) / n_se / (us * 1e3)
        gr = sum(d.get("GRBM_GUI_ACTIVE", 0.0) for d in ds) / len(ds) / n_xcc / (us * 1e3)
        print(f"| `{label}` | {len(ds)} | {us:.1f} | {f32:.2f} | {bf:.2f} | {xf:.2f} | {f32 / us * 1e3:.1f} | "
              f"{sq:.3f} | {gr:.3f} |")


def configs_summary(path, warmup, steps):
    """Per (kernel, grid size): the mean duration of the timed core dispatches
    of each configuration in a kernel trace of --configs-only: the first
    section after a settle loop in which that configuration's chunk-intra
    launch shape appears (the layer's own launches of the same shape come in
    later sections and are not counted), warm-up launches skipped."""
    import csv

    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    groups, owner = {}, {}
    for si, sec in enumerate(_timed_sections(rows)):
        cur = None  # the configuration, known by the shape of its chunk-intra launch
        for r in sec:
            key = (_short(r["Kernel_Name"]), int(r.get("Grid_Size", r.get("Grid_Size_X", 0)) or 0))
            if not key[0].startswith(("chunk_intra", "chunk_inter", "chunk_chain")):
                continue
            if key[0].startswith("chunk_intra"):
                cur = key
            g = (cur,) + key
            if owner.setdefault(g, si) != si:
                continue
            groups.setdefault(g, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print("| configuration (its chunk-intra launch) | kernel | grid (work-items) | timed dispatches | mean us | "
          "min us | max us |")
    print("|---|---|---|---|---|---|---|")
    for (c, name, grid), d in groups.items():
        d = d[warmup:warmup + steps]
        if d:
            print(f"| `{c[0]}` x {c[1] // 512} | `{name}` | {grid} | {len(d)} | {sum(d) / len(d):.1f} | {min(d):.1f} | "
                  f"{max(d):.1f} |")


def layer_gemm_tflop(cfg, tokens):
    """Input-side, gate and o_proj GEMM TFLOP of one forward over `tokens`."""
    V = cfg.v_head
    g_in = 2 * tokens * cfg.hidden_size * (3 * cfg.kd + 2 * cfg.vd + 2 * V) / 1e12
    g_gate = 2 * tokens * V * (cfg.kd + cfg.vd) / 1e12
    g_out = 2 * tokens * cfg.vd * cfg.hidden_size / 1e12
    return g_in, g_gate, g_out


def time_train_steps(torch, G, layer, x, gen, args, recompute):
    """One training step: forward_train keeping its activations, then the
    backward into persistent parameter gradients and dx (d_out ~ N(0,1));
    with `recompute` also the variant whose backward recomputes the forward."""
    B, T = x.shape[:2]
    tokens = B * T
    g_in, g_gate, g_out = layer_gemm_tflop(layer.config, tokens)
    d_out = torch.randn(x.shape, generator=gen, device=x.device, dtype=torch.float32)
    grads = G.Gdn2Grads(layer)
    acts = G.Gdn2Saved(layer, B, T)

    def train_step():
        layer.forward_train(x, saved=acts)
        layer.backward(x, d_out, grads=grads, saved=acts)

    res = {}
    tr = time_layer(torch, train_step, args.layer_steps, tokens, args.settle_ms)
    tr["gemm_tflop"] = 3 * (g_in + g_gate + g_out)
    tr["activations"] = "saved by forward_train"
    res["train_step"] = tr
    acts.close()
    if recompute:
        def train_step_recompute():
            layer.forward_train(x)
            layer.backward(x, d_out, grads=grads)

        rc = time_layer(torch, train_step_recompute, args.layer_steps, tokens, args.settle_ms)
        rc["gemm_tflop"] = 4 * (g_in + g_gate) + 3 * g_out
        rc["activations"] = "recomputed by the backward"
        res["train_step_recompute"] = rc
    grads.close()
    return res


def time_layer(torch, fn, steps, tokens, settle_ms):
    """Whole-layer forward calls (Linear GEMMs + kernels) timed with events."""
    settle(torch, fn, settle_ms)
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"ms_per_step": ms, "tokens_per_s": tokens / (ms / 1e3), "steps": steps}


def time_decode_kernel(torch, G, dev, cfg, Bd, steps, nrot, settle_ms, seed=43):
    """The fused decode kernel (gdn2_decode_fused_f32) alone for layer config
    cfg at batch Bd: `steps` tokens whose raw projections are prepared up
    front, nrot rotating state buffers (the kernel's time does not depend on
    the state values), timed with events on the launch stream after a settle
    loop; beside it a streaming copy of the same bytes.  Bytes per step: the
    state read and written, the raw projections and gate in, the conv caches
    read and written, the output, the per-channel parameters."""
    import ctypes

    from gdn2_amd import _capi as CA
    from gdn2_amd.ops import _stream, decode_args

    H, HV, K, V = cfg.num_heads, cfg.hv, cfg.head_dim, cfg.v_head
    kd, vd = cfg.kd, cfg.vd
    Wn = G.init_params(cfg, seed=1337)
    W = {n: torch.from_numpy(a).to(dev) for n, a in Wn.items() if a is not None}
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    x = torch.randn((steps, Bd, cfg.hidden_size), generator=gen, device=dev)
    with torch.no_grad():
        raw = {"q_raw": x @ W["q_proj"], "k_raw": x @ W["k_proj"], "v_raw": x @ W["v_proj"],
               "f_raw": (x @ W["f_proj_0"]) @ W["f_proj_1"], "b_raw": x @ W["b_proj"], "w_raw": x @ W["w_proj"],
               "gate": (x @ W["g_proj_0"]) @ W["g_proj_1"] + W["g_proj_1_bias"]}
    states = [torch.randn((Bd, HV, K, V), generator=gen, device=dev) * 0.05 for _ in range(nrot)]
    conv = [tuple(torch.randn((Bd, 3, n), generator=gen, device=dev) for n in (kd, kd, vd)) for _ in range(2)]
    out = torch.empty((Bd, vd), device=dev)
    pnames = ("q_conv_w", "k_conv_w", "v_conv_w", "a_log", "dt_bias", "o_norm_weight") + \
        (("decay_factors",) if cfg.min_decay is not None else ())
    params = {n: W[n] for n in pnames}
    blocks = [decode_args({n: a[t] for n, a in raw.items()}, params, states[t % nrot], conv[t % 2],
                          conv[(t + 1) % 2], out, num_heads=H, num_v_heads=HV, head_dim=K, head_v_dim=V,
                          scale=K ** -0.5, min_decay=cfg.min_decay, norm_eps=cfg.norm_eps,
                          allow_neg_eigval=cfg.allow_neg_eigval) for t in range(steps)]
    L, stream = CA.lib(), _stream()
    fn = L.gdn2_decode_fused_f32
    it = [0]

    def one_step():  # cycles through the prepared tokens and rotating buffers
        CA.check(fn(ctypes.byref(blocks[it[0] % steps]), stream))
        it[0] += 1

    settle(torch, one_step, settle_ms)
    for t in range(min(8, steps)):
        CA.check(fn(ctypes.byref(blocks[t]), stream))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for t in range(steps):
        fn(ctypes.byref(blocks[t]), stream)
    e1.record()
    torch.cuda.synchronize()
    CA.check(fn(ctypes.byref(blocks[0]), stream))  # surfaces any launch error of the timed loop
    ms = e0.elapsed_time(e1) / steps
    state_bytes = 2 * Bd * HV * K * V * 4
    io_bytes = Bd * (4 * kd + 3 * vd) * 4 + 2 * Bd * 3 * (2 * kd + vd) * 4 + Bd * vd * 4
    param_bytes = (4 * (2 * kd + vd) + H + kd + V + (kd if cfg.min_decay is not None else 0)) * 4
    bytes_step = state_bytes + io_bytes + param_bytes
    gbs = bytes_step / (ms / 1e3) / 1e9
    copy_same = decode_copy_roof(torch, dev, bytes_step, steps, nrot)
    del blocks, states, conv, raw, x, W
    torch.cuda.empty_cache()
    return {"batch": Bd, "tokens_per_s": Bd / (ms / 1e3), "ms_per_token_step": ms, "bytes_per_step": bytes_step,
            "core_bytes_per_step": 2 * Bd * HV * K * V * 4 + Bd * (4 * HV * K + 3 * HV * V) * 4,
            "achieved_GBs": gbs, "peak_GBs": PEAK_HBM_GBS, "frac_hbm": gbs / PEAK_HBM_GBS,
            "rotating_state_buffers": nrot, "kernel": "gdn2_decode_fused_f32",
            "copy_same_bytes": copy_same, "frac_copy_same_bytes": copy_same["us"] / (ms * 1e3)}


def bench_step(torch, G, args, dev):
    """The bare one-token step (gdn2_recurrent_step_f32, the reference's
    fused_step) at B = 64, 16 heads, K = V = 128: `decode_steps` tokens of
    q, k, g, b [B, H, K] and v, w [B, H, V] prepared up front (L2-normalised
    k, g in [-0.3, -0.02]), the state updated in place in `decode_rotate`
    rotating buffers, timed with events on the launch stream; beside it a
    streaming copy of the same bytes.  Bytes per step: the state read and
    written plus q, k, g, b, v, w in and the output (2 B HV K V 4 +
    B (4 HV K + 3 HV V) 4)."""
    import ctypes

    from gdn2_amd import _capi as CA
    from gdn2_amd.ops import _stream

    B, H, K, V = args.decode_batch, 16, 128, 128
    steps, nrot = args.decode_steps, max(1, args.decode_rotate)
    gen = torch.Generator(device=dev)
    gen.manual_seed(47)
    q = torch.randn((steps, B, H, K), generator=gen, device=dev) * K ** -0.5
    k = torch.nn.functional.normalize(torch.randn((steps, B, H, K), generator=gen, device=dev), dim=-1)
    g = torch.rand((steps, B, H, K), generator=gen, device=dev) * -0.28 - 0.02
    b = torch.rand((steps, B, H, K), generator=gen, device=dev)
    v = torch.randn((steps, B, H, V), generator=gen, device=dev)
    w = torch.randn((steps, B, H, V), generator=gen, device=dev)
    states = [torch.randn((B, H, K, V), generator=gen, device=dev) * 0.05 for _ in range(nrot)]
    out = torch.empty((B, H, V), device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    blocks = [CA.StepArgs(P(q[t]), P(k[t]), P(g[t]), P(b[t]), P(v[t]), P(w[t]), P(states[t % nrot]),
                          P(states[t % nrot]), P(out), B, H, H, K, V, H * K, K, H * V, V, H * V, V, K ** -0.5)
              for t in range(steps)]
    L, stream = CA.lib(), _stream()
    fn = L.gdn2_recurrent_step_f32
    it = [0]

    def one_step():
        CA.check(fn(ctypes.byref(blocks[it[0] % steps]), stream))
        it[0] += 1

    settle(torch, one_step, args.settle_ms)
    for t in range(min(8, steps)):
        CA.check(fn(ctypes.byref(blocks[t]), stream))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for t in range(steps):
        fn(ctypes.byref(blocks[t]), stream)
    e1.record()
    torch.cuda.synchronize()
    CA.check(fn(ctypes.byref(blocks[0]), stream))
    ms = e0.elapsed_time(e1) / steps
    bytes_step = 2 * B * H * K * V * 4 + B * (4 * H * K + 3 * H * V) * 4
    gbs = bytes_step / (ms / 1e3) / 1e9
    copy_same = decode_copy_roof(torch, dev, bytes_step, steps, nrot)
    del blocks, states, q, k, g, b, v, w, out
    torch.cuda.empty_cache()
    tr = load_traffic("step_b64_traffic.json") if B == 64 else None
    return {"workload": f"bare one-token step (fused_step), B={B} H=16 K=V=128, state in place",
            "traffic": None if tr is None else tr.get("hbm_bytes_per_launch"),
            "kernel": "gdn2_recurrent_step_f32", "batch": B, "tokens_per_s": B / (ms / 1e3),
            "ms_per_token_step": ms, "bytes_per_step": bytes_step, "achieved_GBs": gbs, "peak_GBs": PEAK_HBM_GBS,
            "frac_hbm": gbs / PEAK_HBM_GBS, "rotating_state_buffers": nrot, "copy_same_bytes": copy_same,
            "frac_copy_same_bytes": copy_same["us"] / (ms * 1e3)}


def bench_decode(torch, G, args, dev):
    """Config 3: the default layer (FusedRecurrent, short conv) at B = 64.
    (a) The fused decode kernel alone over 256 tokens whose raw projections
    are prepared up front, with rotating state buffers (larger than the
    256 MB MALL; the kernel's time does not depend on the state values).
    (b) The whole layer: forward() over a 2048-token prefill, then 256
    single-token forward() calls carrying the Gdn2State.
    (c) The fused decode kernel at the GVA + extensions configuration (C4:
    8 key heads, 16 value heads, K 128, V 256, neg-eig, min_decay) at its
    batch of 4."""
    cfg = G.Gdn2Config(hidden_size=2048, num_heads=16, head_dim=128, expand_v=1.0)
    Bd = args.decode_batch
    steps = args.decode_steps
    nrot = max(1, args.decode_rotate)
    res = time_decode_kernel(torch, G, dev, cfg, Bd, steps, nrot, args.settle_ms)
    tr = load_traffic("decode_b64_traffic.json") if Bd == 64 else None
    res["traffic"] = None if tr is None else tr.get("hbm_bytes_per_launch")
    over, B4 = OTHER_CONFIGS["C4"][0], OTHER_CONFIGS["C4"][1]
    cfg4 = G.Gdn2Config(**dict(over, mode="fused_recurrent"))
    # as many rotating states as the B = 64 leg's bytes (more than the 256 MB MALL)
    nrot4 = max(nrot, -(-nrot * Bd * cfg.hv * cfg.head_dim * cfg.v_head // (B4 * cfg4.hv * cfg4.head_dim * cfg4.v_head)))
    c4 = time_decode_kernel(torch, G, dev, cfg4, B4, steps, nrot4, args.settle_ms, seed=48)
    c4["workload"] = "C4 decode: " + OTHER_CONFIGS["C4"][5]
    res["c4_decode"] = c4
    gen = torch.Generator(device=dev)
    gen.manual_seed(49)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if not args.no_layer:
        layer = G.GatedDeltaNet2(cfg, seed=1337)
        xp = torch.randn((Bd, args.decode_prefill, cfg.hidden_size), generator=gen, device=dev)
        xs = torch.randn((steps, Bd, 1, cfg.hidden_size), generator=gen, device=dev)
        layer.forward(xp)  # first call of this shape: workspace and GEMM plans
        torch.cuda.synchronize()
        e0.record()
        _, st = layer.forward(xp)
        e1.record()
        torch.cuda.synchronize()
        pre_ms = e0.elapsed_time(e1)
        del xp
        sd = [st, 0]

        def one_token():  # the state keeps evolving; its values do not change the timing
            sd[0] = layer.forward(xs[sd[1] % steps], sd[0])[1]
            sd[1] += 1

        settle(torch, one_token, args.settle_ms)
        st = sd[0]
        for t in range(min(4, steps)):  # warm-up, then restart from the prefill state is not needed for timing
            _, st = layer.forward(xs[t], st)
        torch.cuda.synchronize()
        e0.record()
        for t in range(steps):
            _, st = layer.forward(xs[t], st)
        e1.record()
        torch.cuda.synchronize()
        lms = e0.elapsed_time(e1) / steps
        res["layer"] = {"prefill_tokens": Bd * args.decode_prefill, "prefill_ms": pre_ms,
                        "prefill_tokens_per_s": Bd * args.decode_prefill / (pre_ms / 1e3),
                        "decode_ms_per_token_step": lms, "decode_tokens_per_s": Bd / (lms / 1e3),
                        "weight_bytes_per_step": sum(a.nbytes for a in layer.params().values() if a is not None)}
        del st
        layer.close()
    return res


def cpu_baseline(pre, args):
    """The oracle's f32 restatement of chunk_wy_forward (the reference's
    Chunk-mode tensor path) on the host cores, on the first cpu_batch
    sequences of the same projected inputs."""
    from oracle import oracle as O

    hs = pre["host_sample"]
    n = hs["q"].shape[0]
    O.chunk_wy_f32(*(a[:, :, :256] for a in (hs["q"], hs["k"], hs["v"], hs["g"], hs["b"], hs["w"])),
                   scale=pre["scale"], chunk_size=64)  # warm-up
    t0 = time.perf_counter()
    O.chunk_wy_f32(hs["q"], hs["k"], hs["v"], hs["g"], hs["b"], hs["w"], scale=pre["scale"], chunk_size=64)
    dt = time.perf_counter() - t0
    T = hs["q"].shape[2]
    cores = O.num_threads()
    return {"value": n * T / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} of 8 sequences x {T} tokens x 16 heads, f32 chunk_wy_forward restatement "
                      f"(oracle/gdn2_oracle.c), {cores} OpenMP threads, {dt:.2f} s",
            "cpu_model": _cpu_model(), "layer": cpu_layer_baseline(args), "decode_b64": cpu_decode_core(args)}


def cpu_config_core(name, host, scale):
    """The recurrence core of one batch row of a configuration on the host
    cores: the oracle's f32 restatement of chunk_wy_forward (the Chunk-mode
    tensor path), except for the long-context configuration, where the
    reference's chunked tensor path overflows (its decay factor
    k / exp(G_s - G_b) passes the f32 range once 16 |g| > 88), so its f32
    per-token scan (fused_recurrent_forward) is timed instead."""
    from oracle import oracle as O

    q, k, v, g, b, w = host
    T = q.shape[2]
    short = [a[:, :, :min(T, 128)] for a in host]
    if name == "C5":
        fn, what = O.recurrent_f32, "f32 per-token scan restatement (fused_recurrent_forward)"
        fn(*short, scale=scale)
        t0 = time.perf_counter()
        fn(q, k, v, g, b, w, scale=scale)
    else:
        fn, what = O.chunk_wy_f32, "f32 chunk_wy_forward restatement"
        fn(*short, scale=scale, chunk_size=64)
        t0 = time.perf_counter()
        fn(q, k, v, g, b, w, scale=scale, chunk_size=64)
    dt = time.perf_counter() - t0
    cores = O.num_threads()
    return {"value": T / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"1 batch row x {T} tokens x {v.shape[1]} value heads, {what} (oracle/gdn2_oracle.c), "
                      f"{cores} OpenMP threads, {dt:.2f} s"}


def cpu_decode_core(args):
    """One B = 64 decode step of the recurrence core on the host cores: the
    oracle's f32 per-token scan over one token for 64 x 16 heads (K = V =
    128), averaged over 20 steps."""
    import numpy as np

    from oracle import oracle as O

    rng = np.random.default_rng(7)
    B, H, K, V = args.decode_batch, 16, 128, 128
    q = rng.standard_normal((B, H, 1, K)).astype(np.float32)
    kk = rng.standard_normal((B, H, 1, K))
    k = (kk / np.linalg.norm(kk, axis=-1, keepdims=True)).astype(np.float32)
    v, w = (rng.standard_normal((B, H, 1, V)).astype(np.float32) for _ in range(2))
    g = rng.uniform(-0.3, -0.02, (B, H, 1, K)).astype(np.float32)
    b = rng.uniform(0, 1, (B, H, 1, K)).astype(np.float32)
    S = (rng.standard_normal((B, H, K, V)) * 0.05).astype(np.float32)
    O.recurrent_f32(q, k, v, g, b, w, S0=S, scale=K ** -0.5)
    n = 20
    t0 = time.perf_counter()
    for _ in range(n):
        O.recurrent_f32(q, k, v, g, b, w, S0=S, scale=K ** -0.5)
    dt = (time.perf_counter() - t0) / n
    cores = O.num_threads()
    return {"value": B / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"B={B} one-token steps x 16 heads, f32 per-token scan restatement (oracle), {cores} OpenMP "
                      f"threads, {n} steps of {dt * 1e3:.2f} ms"}


def cpu_layer_baseline(args):
    """The whole layer's forward_train on the host cores, the way the
    reference's CPU backend computes it (f32 Linear layers through BLAS sgemm,
    the gates and norms, chunk_wy_forward as the core), on one sequence of
    cpu_layer_tokens tokens of the benchmarked layer (D=2048, H=16, K=V=128)."""
    import numpy as np

    import gdn2_amd as G
    from oracle import oracle as O

    cfg = G.Gdn2Config(hidden_size=2048, num_heads=16, head_dim=128, expand_v=1.0, mode="chunk", chunk_size=64)
    W = G.init_params(cfg, seed=1337)
    T = args.cpu_layer_tokens
    x = np.random.default_rng(42).standard_normal((1, T, cfg.hidden_size)).astype(np.float32)
    O.layer_forward_f32_host(cfg, W, x[:, :64])  # warm-up
    t0 = time.perf_counter()
    O.layer_forward_f32_host(cfg, W, x)
    dt = time.perf_counter() - t0
    return {"value": T / dt, "unit": "tokens/s", "cores": O.num_threads(), "kind": "port",
            "sample": f"1 sequence x {T} tokens of the D=2048 layer's forward_train: numpy f32 sgemm Linear layers "
                      f"+ numpy f32 glue + f32 chunk_wy_forward restatement (oracle), {dt:.2f} s"}


def _median(xs):
    ys = sorted(xs)
    n = len(ys)
    return ys[n // 2] if n % 2 else 0.5 * (ys[n // 2 - 1] + ys[n // 2])


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


COPY_BYTES = 1 << 30
# the inference instances at the benchmarked shape (the training variants,
# chunk_intra_kernel<..., true> and chunk_inter_kernel<128, 2 or 4, 4>, are others)
KERNELS = {"chunk_intra": "chunk_intra_kernel<128, 128, false>", "chunk_inter": "chunk_inter_kernel<128, 0, 4>",
           "decode": "decode_fused_kernel<128, 128>", "step": "step_kernel<128, 128>"}
BWD_KERNELS = ("chunk_intra_kernel<128, 128, true>", "chunk_inter_kernel<128, 2, 4>", "chunk_inter_kernel<128, 4, 4>",
               "bwd_inter_kernel<128, 0, 4>", "bwd_vprod_kernel<128, 128>", "bwd_decay_kernel<128, 128>")


def _short(name):
    import re

    m = re.search(r"(?:gdn2::)?\(anonymous namespace\)::(\w+(<[^>]*>)?)", name)
    if m:
        return m.group(1)
    return name.split("(")[0].replace("void ", "")[:70]


def stats_summary(path):
    """The library's kernels by total time; hipBLASLt's GEMM kernels (the
    layer's Linear layers, many kernel names, including the candidates timed
    on the first call of each shape) are summed into one row."""
    import csv

    rows = list(csv.DictReader(open(path)))
    gemm = [r for r in rows if r["Name"].startswith("Cijk")]
    own = [r for r in rows if not r["Name"].startswith("Cijk")]
    print("| kernel | calls | avg us | total us | % of GPU time |")
    print("|---|---|---|---|---|")
    for r in sorted(own, key=lambda r: -float(r["TotalDurationNs"]))[:12]:
        print(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
              f"{float(r['TotalDurationNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
    if gemm:
        calls = sum(int(r["Calls"]) for r in gemm)
        tot = sum(float(r["TotalDurationNs"]) for r in gemm)
        pct = sum(float(r["Percentage"]) for r in gemm)
        print(f"| hipBLASLt GEMM kernels ({len(gemm)} names) | {calls} | {tot / calls / 1e3:.1f} | {tot / 1e3:.1f} | "
              f"{pct:.1f} |")


def _timed_sections(rows):
    """Splits launch-ordered trace rows at the settle markers (see mark()):
    a section starts at a tail_copy_kernel launch (end of a settle loop) and
    ends at the next stream_copy_kernel or tail_copy_kernel launch; the rows
    of each section are the warm-up and timed dispatches of one workload.
    Returns a list of row lists."""
    sections, cur = [], None
    for r in rows:
        name = _short(r["Kernel_Name"])
        if name in ("stream_copy_kernel", "tail_copy_kernel"):
            if cur is not None:
                sections.append(cur)
            cur = [] if name == "tail_copy_kernel" else None
        elif cur is not None:
            cur.append(r)
    if cur is not None:
        sections.append(cur)
    return sections


def timed_summary(path, warmup, steps, decode_steps):
    """The timed dispatches of the prefill core (in the first section after a
    settle loop that launches each kernel: warmup launches skipped, then
    steps) and of the decode kernel (eight warm-up launches, then
    decode_steps), as the bench line's kernel times see them."""
    import csv

    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    sections = _timed_sections(rows)
    print("| kernel | timed dispatches | mean us | min us | max us |")
    print("|---|---|---|---|---|")
    for label, key, skip, take in (("chunk_intra", "chunk_intra_kernel<128, 128, false>", warmup, steps),
                                   ("chunk_inter", "chunk_inter_kernel<128, 0, 4>", warmup, steps),
                                   ("decode", "decode_fused_kernel<128, 128>", 8, decode_steps),
                                   ("decode C4", "decode_fused_kernel<128, 256>", 8, decode_steps),
                                   ("bare step", "step_kernel<128, 128>", 8, decode_steps)):
        for sec in sections:
            d = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in sec
                 if _short(r["Kernel_Name"]) == key]
            if d:
                d = d[skip:skip + take]
                if d:
                    print(f"| `{key}` ({label}) | {len(d)} | {sum(d) / len(d):.1f} | {min(d):.1f} | {max(d):.1f} |")
                break


def backward_summary(path):
    """The sections (see _timed_sections) of the backward entries: the
    recomputing backward, the training forward and the saved backward of each
    configuration timed with its backward, in launch order.  One line per
    section: each chunk / backward kernel's mean duration and dispatch count,
    and their sum (one call)."""
    import csv

    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    kinds = ("bwd_", "chunk_intra_kernel<", "chunk_inter_kernel<", "chunk_chain_kernel<")
    for si, sec in enumerate(_timed_sections(rows)):
        names = [_short(r["Kernel_Name"]) for r in sec]
        # the backward's sections: a backward kernel, or the training variants of the forward,
        # from the section's first dispatch on (the layer's sections start with its GEMMs;
        # the next workload's set-up can follow in the same section)
        train = any(n.startswith("bwd_") or (n.startswith("chunk_intra_kernel<") and n.endswith("true>"))
                    for n in names)
        if not train or not names or not names[0].startswith(kinds):
            continue
        acc, order = {}, []
        for r, n in zip(sec, names):
            if not n.startswith(kinds):
                break  # the end of the backward entry's dispatches
            if n not in acc:
                order.append(n)
            acc.setdefault(n, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        tot = sum(sum(d) / len(d) for d in acc.values())
        print(f"section {si}: " + ", ".join(f"`{n}` {sum(acc[n]) / len(acc[n]):.1f} (x{len(acc[n])})" for n in order)
              + f"; sum {tot:.1f} us")


def train_summary(path):
    """The kernels of the last training step of a --train-only trace: from the
    forward's input GEMM (the long GEMM before its project_kernel) to the end."""
    import csv
    import re

    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    last = max(i for i, r in enumerate(rows) if "project_kernel" in r["Kernel_Name"])
    # the step starts at the input GEMM: walk back over the GEMM and fill
    # launches before project_kernel up to the first long (> 1 ms) GEMM, which
    # is x W_in; the one before it is the previous step's dx GEMM
    start, big = last, 0
    for i in range(last - 1, -1, -1):
        name = rows[i]["Kernel_Name"]
        if not (name.startswith("Cijk") or "fill_rows" in name):
            break
        if int(rows[i]["End_Timestamp"]) - int(rows[i]["Start_Timestamp"]) > 1_000_000:
            big += 1
            if big > 1:
                break
        start = i
    step = rows[start:]
    t0 = int(step[0]["Start_Timestamp"])
    print("| start us | duration us | kernel |")
    print("|---|---|---|")
    gemm = other = 0.0
    for r in step:
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        name = r["Kernel_Name"]
        if name.startswith("Cijk"):
            m = re.search(r"MT\d+x\d+x\d+", name)
            label = f"hipBLASLt {name[:14]} {m.group(0) if m else ''}"
            gemm += d
        else:
            label = _short(name)
            other += d
        print(f"| {(int(r['Start_Timestamp']) - t0) / 1e3:.1f} | {d:.1f} | `{label}` |")
    span = (int(step[-1]["End_Timestamp"]) - t0) / 1e3
    print(f"\nspan {span:.1f} us; GEMM kernels {gemm:.1f} us, other kernels {other:.1f} us")


def mix_summary(csv1, csv2, n_xcc=8, n_simd=1024):
    """Per dispatch of each timed kernel, counters summed over the chip, then
    averaged over its dispatches: instructions per wave, MFMA busy =
    SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / n_xcc x n_simd), waiting =
    SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES."""
    import csv

    kernels = dict(KERNELS, bwd_inter=BWD_KERNELS[3], bwd_vprod=BWD_KERNELS[4], bwd_decay=BWD_KERNELS[5])
    per = {}
    for path in (csv1, csv2):
        for r in csv.DictReader(open(path)):
            for key, frag in kernels.items():
                if frag in r["Kernel_Name"]:
                    d = per.setdefault(key, {}).setdefault(r["Dispatch_Id"], {})
                    d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])

    def mean(key, name, scale=None):
        vals = [d[name] / (d[scale] if scale else 1.0) for d in per[key].values() if name in d and (not scale or d.get(scale))]
        return sum(vals) / len(vals) if vals else float("nan")

    print("| kernel | waves | VALU | MFMA | SALU | LDS | VMEM rd / wr | MFMA busy (per SIMD) | wave cycles waiting |")
    print("|---|---|---|---|---|---|---|---|---|")
    for key in kernels:
        if key not in per:
            continue
        waves = mean(key, "SQ_WAVES")
        busy = [d["SQ_VALU_MFMA_BUSY_CYCLES"] / (d["GRBM_GUI_ACTIVE"] / n_xcc * n_simd)
                for d in per[key].values() if d.get("GRBM_GUI_ACTIVE") and "SQ_VALU_MFMA_BUSY_CYCLES" in d]
        busy_s = f"{100 * sum(busy) / len(busy):.1f} %" if busy and key not in ("decode", "step") else "-"
        wait = mean(key, "SQ_WAIT_INST_ANY") / mean(key, "SQ_WAVE_CYCLES")
        pw = lambda n: mean(key, n) / waves
        print(f"| {key} | {waves:.0f} | {pw('SQ_INSTS_VALU'):.0f} | {pw('SQ_INSTS_MFMA'):.0f} | {pw('SQ_INSTS_SALU'):.0f} | "
              f"{pw('SQ_INSTS_LDS'):.0f} | {pw('SQ_INSTS_VMEM_RD'):.0f} / {pw('SQ_INSTS_VMEM_WR'):.0f} | {busy_s} | "
              f"{100 * wait:.0f} % |")


def _tagged(name, frag):
    """frag in the kernel name; a frag ending in a " (tag)" also needs the tag."""
    if frag.endswith(")"):
        base, tag = frag.rsplit(" (", 1)
        return base in name and name.endswith(" (" + tag)
    return frag in name


def traffic_summary(fetch_csv, write_csv):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) per kernel, scaled so that
    the 1 GiB streaming copy (gdn2_stream_copy_f32) reads and writes 1 GiB."""
    import csv

    def per_kernel(path, counter):
        # the training chunk-intra serves the recomputing backward (followed by
        # the states pass) and the training forward (followed by its output
        # pass): its dispatches are named by the kernel that follows them
        rows = sorted((r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter),
                      key=lambda r: int(r["Dispatch_Id"]))
        acc = {}
        for i, r in enumerate(rows):
            name = r["Kernel_Name"]
            if BWD_KERNELS[0] in _short(name) and i + 1 < len(rows):
                nxt = _short(rows[i + 1]["Kernel_Name"])
                name += " (recompute)" if BWD_KERNELS[1] in nxt else " (training forward)" if BWD_KERNELS[2] in nxt else ""
            acc.setdefault(name, []).append(float(r["Counter_Value"]) * 1024.0)
        return acc

    fetch, write = per_kernel(fetch_csv, "FETCH_SIZE"), per_kernel(write_csv, "WRITE_SIZE")

    def copy_bytes(acc):
        # the largest dispatch of the library's streaming copy is the 1 GiB
        # copy of the measured roof (torch's own kernels of the run read other
        # sizes, e.g. comparisons of two 1 GiB tensors)
        best = 0.0
        for name, vals in acc.items():
            if "stream_copy_kernel" in name:
                best = max(best, max(vals))
        return best

    f_fac = COPY_BYTES / copy_bytes(fetch)
    w_fac = COPY_BYTES / copy_bytes(write)
    print(f"calibration: FETCH_SIZE x {f_fac:.3f}, WRITE_SIZE x {w_fac:.3f} (1 GiB copy)")
    print("| kernel | dispatches | HBM read GB/launch | HBM write GB/launch | total GB/launch |")
    print("|---|---|---|---|---|")
    out = {}
    for key, frag in KERNELS.items():
        fv = [v for n, vals in fetch.items() if frag in n for v in vals]
        wv = [v for n, vals in write.items() if frag in n for v in vals]
        if not fv or not wv:
            continue
        rd, wr = sum(fv) / len(fv) * f_fac, sum(wv) / len(wv) * w_fac
        out[key] = {"hbm_bytes_per_launch": rd + wr, "read_bytes": rd, "write_bytes": wr,
                    "dispatches": len(fv), "fetch_factor": f_fac, "write_factor": w_fac}
        print(f"| `{key}` | {len(fv)} | {rd / 1e9:.3f} | {wr / 1e9:.3f} | {(rd + wr) / 1e9:.3f} |")
        suffix = "b64" if key in ("decode", "step") else "b8_t4096"
        with open(os.path.join(ROOT, "profiles", f"{key}_{suffix}_traffic.json"), "w") as fh:
            json.dump(out[key], fh, indent=1)
    # the chunked backward's kernels (bench.py's backward entry), printed only
    bwd = [BWD_KERNELS[0] + " (recompute)", BWD_KERNELS[1], BWD_KERNELS[0] + " (training forward)"] + list(BWD_KERNELS[2:])
    for frag in bwd:
        fv = [v for n, vals in fetch.items() if _tagged(n, frag) for v in vals]
        wv = [v for n, vals in write.items() if _tagged(n, frag) for v in vals]
        if fv and wv:
            rd, wr = sum(fv) / len(fv) * f_fac, sum(wv) / len(wv) * w_fac
            print(f"| `{frag}` | {len(fv)} | {rd / 1e9:.3f} | {wr / 1e9:.3f} | {(rd + wr) / 1e9:.3f} |")
    return out


def time_chunk_backward(torch, args, dev, q, k, g, b, v, w, label, scan=False):
    """gdn2_chunk_bwd_f32 on the given operands (d_out ~ N(0,1)): the
    gradients of q, k, g, b, v, w and S0, recomputing the forward's per-chunk
    quantities; then gdn2_chunk_fwd_train_f32 (the forward keeping them) and
    gdn2_chunk_bwd_saved_f32 (the backward reading them).  scan: also the
    per-token scan's adjoint (gdn2_recurrent_bwd_f32) on the same operands.
    Outputs and the workspaces are allocated before the timed regions."""
    import ctypes

    from gdn2_amd import _capi as CA
    from gdn2_amd.ops import _p, _stream, chunk_args

    B, H, T, K = q.shape
    V = v.shape[3]
    gen = torch.Generator(device=dev)
    gen.manual_seed(44)
    S0 = torch.zeros((B, H, K, V), device=dev)
    dO = torch.randn((B, H, T, V), generator=gen, device=dev)
    grads = [torch.empty_like(t) for t in (q, k, g, b, v, w)] + [torch.empty_like(S0)]
    fwd = chunk_args(q, k, v, g, b, w, S0, dO, K ** -0.5, 64)
    a = CA.ChunkBwdArgs(fwd, _p(dO), None, *(_p(t) for t in grads), None, 0)
    L = CA.lib()
    need = int(L.gdn2_chunk_bwd_workspace_bytes(ctypes.byref(a)))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = _p(ws), need
    stream = _stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, n):
        settle(torch, fn, args.settle_ms)
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    pa = ctypes.byref(a)
    ms = timed(lambda: CA.check(L.gdn2_chunk_bwd_f32(pa, stream)), args.steps)
    res = {"workload": f"chunked backward (gradients of q, k, g, b, v, w, S0), {label}",
           "ms_per_step": ms, "tokens_per_s": B * T / (ms / 1e3), "workspace_bytes": need,
           "kernel": "gdn2_chunk_bwd_f32"}

    # the training forward (output + final state, keeping the backward's inputs
    # in the workspace), then the backward from them
    St = torch.zeros_like(S0)
    out = torch.empty((B, T, H, V), device=dev).permute(0, 2, 1, 3)
    at = CA.ChunkBwdArgs(chunk_args(q, k, v, g, b, w, St, out, K ** -0.5, 64), _p(dO), None,
                         *(_p(t) for t in grads), _p(ws), need)
    pt = ctypes.byref(at)
    fwd_ms = timed(lambda: CA.check(L.gdn2_chunk_fwd_train_f32(pt, stream)), args.steps)
    saved_ms = timed(lambda: CA.check(L.gdn2_chunk_bwd_saved_f32(pt, stream)), args.steps)
    res["from_saved_forward"] = {
        "kernel": "gdn2_chunk_bwd_saved_f32", "ms_per_step": saved_ms, "tokens_per_s": B * T / (saved_ms / 1e3),
        "training_forward": {"kernel": "gdn2_chunk_fwd_train_f32", "ms_per_step": fwd_ms,
                             "tokens_per_s": B * T / (fwd_ms / 1e3)},
        "what": "the backward reading the training forward's per-chunk quantities instead of recomputing them"}
    if scan:
        from gdn2_amd.ops import _strides3

        rf = CA.RecurrentArgs(_p(q), _p(k), _p(g), _p(b), _p(v), _p(w), _p(S0), None, None, B, q.shape[1], v.shape[1], T, K,
                              V, *_strides3(q), *_strides3(v), *_strides3(dO), K ** -0.5)
        rb = CA.RecurrentBwdArgs(rf, _p(dO), None, *(_p(t) for t in grads), None, 0)
        rneed = int(L.gdn2_recurrent_bwd_workspace_bytes(ctypes.byref(rb)))
        rws = torch.empty(max(rneed, 1), dtype=torch.uint8, device=dev)
        rb.workspace, rb.workspace_bytes = _p(rws), rneed
        prb = ctypes.byref(rb)
        scan_ms = timed(lambda: CA.check(L.gdn2_recurrent_bwd_f32(prb, stream)), max(1, min(args.steps, 5)))
        res["scan"] = {"kernel": "gdn2_recurrent_bwd_f32", "ms_per_step": scan_ms,
                       "tokens_per_s": B * T / (scan_ms / 1e3), "chunk_speedup": scan_ms / ms}
        del rws
    del S0, dO, grads, ws, St, out
    torch.cuda.empty_cache()
    return res


def bench_backward(torch, G, args, dev):
    """The chunked backward on the prefill workload's operands (the layer's
    own project() outputs)."""
    cfg = G.Gdn2Config(hidden_size=2048, num_heads=16, head_dim=128, expand_v=1.0, mode="chunk", chunk_size=64)
    layer = G.GatedDeltaNet2(cfg, seed=1337)
    gen = torch.Generator(device=dev)
    gen.manual_seed(42)
    x = torch.randn((args.batch, args.seq, cfg.hidden_size), generator=gen, device=dev, dtype=torch.float32)
    P = layer.project(x)
    del x
    layer.close()
    res = time_chunk_backward(torch, args, dev, *(P[n] for n in ("q", "k", "g", "b", "v", "w")),
                              f"B={args.batch} T={args.seq} H=16 K=V=128")
    del P
    torch.cuda.empty_cache()
    return res


def main():
    args = parse()
    if args.stats_summary:
        stats_summary(args.stats_summary)
        return
    if args.train_summary:
        train_summary(args.train_summary)
        return
    if args.timed_summary:
        timed_summary(args.timed_summary, args.warmup, args.steps, args.decode_steps)
        return
    if args.backward_summary:
        backward_summary(args.backward_summary)
        return
    if args.traffic_summary:
        traffic_summary(*args.traffic_summary)
        return
    if args.mfma_summary:
        mfma_summary(args.mfma_summary)
        return
    if args.mix_summary:
        mix_summary(*args.mix_summary)
        return
    if args.configs_summary:
        configs_summary(args.configs_summary, args.warmup, args.config_steps)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the GDN-2 path shards over (batch, value head) with no "
              f"communication, so multi-GPU throughput is N x the one-GPU figure; --gpus {args.gpus} "
              f"is not run here.", file=sys.stderr)
        sys.exit(2)
    import torch

    import gdn2_amd as G

    torch.backends.cuda.matmul.allow_tf32 = False
    dev = torch.device("cuda:0")
    if not G.hip_available():
        raise SystemExit("no gfx950 device: bench.py needs an MI355X")
    if args.train_only:
        cfg = G.Gdn2Config(hidden_size=2048, num_heads=16, head_dim=128, expand_v=1.0, mode="chunk", chunk_size=64)
        layer = G.GatedDeltaNet2(cfg, seed=1337)
        gen = torch.Generator(device=dev)
        gen.manual_seed(42)
        x = torch.randn((args.batch, args.seq, cfg.hidden_size), generator=gen, device=dev, dtype=torch.float32)
        res = time_train_steps(torch, G, layer, x, gen, args, recompute=False)
        res["workload"] = f"GDN-2 layer training step, B={args.batch} T={args.seq} D=2048 H=16 K=V=128, f32"
        print(json.dumps(res), flush=True)
        return
    if args.warmup_timeline:
        for r in warmup_timeline(torch, G, args, dev):
            print(json.dumps(r), flush=True)
        return
    if args.configs_only:
        res = {n: bench_other_config(torch, G, args, dev, n) for n in OTHER_CONFIGS}
        res["hbm_copy_roof"] = bench_copy_roof(torch, dev)
        print(json.dumps(res), flush=True)
        return
    pre = bench_prefill(torch, G, args, dev)
    dec = None if args.no_decode else bench_decode(torch, G, args, dev)
    step = None if args.no_decode else bench_step(torch, G, args, dev)
    bwd = None if args.no_backward else bench_backward(torch, G, args, dev)
    others = None if args.no_configs else {n: bench_other_config(torch, G, args, dev, n) for n in OTHER_CONFIGS}
    copy_roof = bench_copy_roof(torch, dev)
    cpu = None if args.no_cpu else cpu_baseline(pre, args)
    if args.copy_calibration:
        src = torch.empty(COPY_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    line = {
        "metric": METRIC,
        "value": pre["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": pre["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: x ~ N(0,1) through seeded random-init layer weights (reference initialisers)",
        "config": {"workload": f"chunked prefill, recurrence core (chunk-intra + chunk-inter), B={args.batch} "
                               f"T={args.seq} H=16 K=V=128 chunk=64",
                   "batch": args.batch, "seq_len": args.seq, "heads": 16, "head_dim": 128, "head_v_dim": 128,
                   "chunk_size": 64},
        "roofline": pre["roofline"],
        "cpu_baseline": cpu,
        "kernels": pre["kernels"],
        "decode": dec,
        "decode_tokens_per_s": None if dec is None else dec["tokens_per_s"],
        "step": step,
        "layer": {"prefill": pre["layer"], "decode": None if dec is None else dec.get("layer")},
        "backward": bwd,
        "configs": others,
        "hbm_copy_roof": copy_roof,
    }
    # fractions of the measured copy bandwidth (the practical HBM roof) beside the 8 TB/s peak
    tr_intra = load_traffic("chunk_intra_b8_t4096_traffic.json") if (args.batch, args.seq) == (8, 4096) else None
    if tr_intra:
        gbs = tr_intra["hbm_bytes_per_launch"] / (pre["kernels"]["chunk_intra"]["ms"] / 1e3) / 1e9
        pre["kernels"]["chunk_intra"].update({"hbm_GBs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS,
                                              "frac_copy_roof": gbs / copy_roof["GBs"]})
    if dec is not None:
        dec["frac_copy_roof"] = dec["achieved_GBs"] / copy_roof["GBs"]
    if step is not None:
        step["frac_copy_roof"] = step["achieved_GBs"] / copy_roof["GBs"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
