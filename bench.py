#!/usr/bin/env python3
"""Benchmark of the SNNtome wave hot path on one MI355X.

Headline workload: the ultra-sparse gather-bound wave — substrate of
40,000,000 positions x batch 256 fp16 (20.5 GB, generated on the device), 65,536 neurons, each
reading 4 dendritic clusters of S=16 consecutive positions (16-aligned uniform starts),
W ~ N(0, 0.05), b ~ N(0, 0.01), ReLU, fp32 accumulation.  One step = one execution of the
compiled one-wave plan through libk44wavec.so (inputs resident in HBM).

Metric: effective TFLOP/s = 2 * nnz * batch / t (nnz = 65,536 x 64 synapses, batch = 256),
reported with the achieved algorithmic HBM GB/s of the wave kernel against the 8 TB/s roofline,
and the CPU path (OpenMP fp32 oracle) timed on the host cores on a bounded sample of the wave.

The default run (no --config) prints ONE JSON line: the headline (config 2) at the top level and
the other BASELINE configurations at their full sizes under "configs" (c1 plumbing, c3 dense
cluster, c4 8-wave plan, c5 LLM-shaped decoder), each with its own binding roofline:
  c1, c4  cache-resident gathers: achieved = gathered bytes / kernel time against the aggregate
          L2 bandwidth (8 XCDs x 16 channels x 128 B/clk x 2.4 GHz = 39.3 TB/s);
  c2, c3  HBM: compulsory (algorithmic) bytes / kernel time against 8 TB/s;
  c5      prefill: effective FLOPs / prefill time against 2.5 PFLOP/s fp16 MFMA; decode: weight
          bytes / step time against HBM.
--config N runs one configuration alone (its record at the top level).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1..5] [--no-cpu] [--graphs]
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
# Aggregate L2 read bandwidth: 8 XCDs x 16 channels x 128 B per clock at 2.4 GHz.
L2_PEAK_GBS = 8 * 16 * 128 * 2.4
METRIC = "effective TFLOP/s (2*nnz*batch) + achieved HBM GB/s per wave, 1xMI355X"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def under_profiler() -> bool:
    """rocprofv3 preloads its tool library into the program it profiles."""
    return "rocprofiler-sdk" in os.environ.get("LD_PRELOAD", "")


def under_counter_collection() -> bool:
    """rocprofv3 --pmc / -i passes the requested counters to its tool through the environment."""
    return under_profiler() and any(
        os.environ.get(k) for k in ("ROCPROF_COUNTER_COLLECTION", "ROCPROF_COUNTERS",
                                    "ROCPROFILER_COUNTERS"))


# Untimed warm-up: the requested warm-up steps, then more until at least this long has passed
# (the reference's sustained warm-up, whitepaper/sparse_wmma_kernel/tests/benchmark_common.cuh:
# 135-161: clocks and caches in their steady state before the timed region).
WARMUP_MIN_S = 0.2
# Config 4 is also timed over this many copies of its plan in rotation (weights and segment
# tables of 4 x 134 MB, beyond the 256 MB last-level cache), as the reference rotates its
# weight and index pools (benchmark_common.cuh:182-190).
C4_POOLS = 4


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def workload(cfg: int):
    from snntome_amd import synth

    return {1: synth.config1, 2: synth.config2, 3: synth.config3, 4: synth.config4}[cfg]()


def traffic_from_profiles(kernel_key: str):
    """HBM bytes per launch measured with rocprofv3 PMC counters (profiles/*.json), if any."""
    p = ROOT / "profiles" / f"{kernel_key}_traffic.json"
    if not p.exists():
        return None
    try:
        return float(json.loads(p.read_text())["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def cpu_baseline(wl, budget_s: float = 12.0, sample_neurons: int = 4096):
    """OpenMP fp32 oracle on a bounded sample of the first wave (same weights / starts),
    gathering from a compact host copy of exactly the substrate rows the sample reads."""
    from oracle import oracle

    w = wl.waves[0]
    n = min(sample_neurons, w.cout)
    n -= n % w.cluster
    rows = n // w.cluster
    stride = (wl.tokens + 63) // 64 * 64
    starts = w.starts[:rows].astype(np.uint64)
    compact = oracle.fill_segments(wl.seed, starts.ravel(), w.S, wl.tokens, stride)
    seg = (np.arange(rows * w.K, dtype=np.uint64) * w.S * stride)
    canvas = np.concatenate([compact.ravel(), np.zeros(n * stride, np.uint16)])
    y_off = compact.size
    threads = len(os.sched_getaffinity(0))
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        used = oracle.wave_f32_omp(canvas, seg, w.weights[:n], w.bias[:n], None, w.K, w.S,
                                   w.cluster, stride, stride, stride, w.act, y_off,
                                   threads=threads)
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    t = float(np.median(times))
    flops = 2.0 * n * w.K * w.S * wl.tokens
    return {
        "value": round(flops / t / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": int(used),
        "kind": "port",
        "cpu_model": cpu_model(),
        "host_threads": os.cpu_count(),
        "sample": (f"{n} of {w.cout} neurons of {w.name} ({n * w.K} segments, "
                   f"{n * w.K * w.S} substrate rows x {wl.tokens} tokens), median of "
                   f"{len(times)} passes, fp32 OpenMP oracle/wave_oracle.c:orc_wave_f32_omp"),
    }


def copy_probe(gib: float):
    """Plain device-to-device copy kernel of known size: the calibration run for the
    FETCH_SIZE / WRITE_SIZE counters (reads and writes exactly n bytes per launch)."""
    import torch

    n = int(gib * (1 << 30))
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[copy-probe] 5 launches of a {n}-byte device copy")


def cpu_baseline_llm(spec, wts, tokens, budget_s: float = 12.0, sample_neurons: int = 256):
    """OpenMP fp32 oracle on a bounded sample of the heaviest projection (layer 0's down
    projection, per-neuron clusters) over the full prefill batch, input from the host generator."""
    from oracle import oracle

    p = wts.proj[0]["dn"]
    n = min(sample_neurons, p.starts.shape[0])
    K = p.starts.shape[1]
    stride = (tokens + 63) // 64 * 64
    x = oracle.fill_substrate(spec.seed, 0, spec.ffn, tokens, stride)
    seg = p.starts[:n].astype(np.uint64).ravel() * np.uint64(stride)
    canvas = np.concatenate([x.ravel(), np.zeros(n * stride, np.uint16)])
    threads = len(os.sched_getaffinity(0))
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        used = oracle.wave_f32_omp(canvas, seg, p.weights[:n], p.bias[:n], None, K, spec.S, 1,
                                   stride, stride, stride, None, x.size, threads=threads)
        times.append(time.perf_counter() - t0)
        if len(times) >= 20:
            break
    t = float(np.median(times))
    return {
        "value": round(2.0 * n * K * spec.S * tokens / t / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": int(used),
        "kind": "port",
        "cpu_model": cpu_model(),
        "host_threads": os.cpu_count(),
        "sample": (f"{n} of {p.starts.shape[0]} neurons of layer 0's down projection "
                   f"({K} x {spec.S} inputs each) x {tokens} prefill tokens, median of "
                   f"{len(times)} passes, fp32 OpenMP oracle/wave_oracle.c:orc_wave_f32_omp"),
    }


def gathered_bytes(wl, w) -> int:
    """Bytes the wave's gathers read (every segment row of every index row x tokens x 2): what a
    cache-resident wave moves from L2 / MALL."""
    stride = (wl.tokens + 63) // 64 * 64
    return 2 * stride * w.starts.size * w.S


def bench_wave(cfg: int, steps: int, warmup: int) -> dict:
    """One of configs 1-4 at full size: compiled plan, device-generated input, `warmup` untimed
    then `steps` timed plan executions bracketed by device synchronisation."""
    from snntome_amd import synth, wavec

    t_start = time.perf_counter()
    wl = workload(cfg)
    log(f"[bench] workload {wl.name}: {wl.description}")
    plan = synth.build_graph(wl, wavec).compile()
    plan.init_gpu()
    plan.fill_input_uniform(wl.seed)
    rep = plan.exec_report()
    for wv in rep["waves"][:2]:
        log(f"[bench] {wv['name']}: path={wv['path']} K={wv['K']} S={wv['S']} "
            f"slab={wv['slab']} tokens={wv['tokens']}")
    log(f"[bench] setup {time.perf_counter() - t_start:.1f}s; warmup {warmup} steps, "
        f">= {WARMUP_MIN_S * 1e3:.0f} ms")
    tw = time.perf_counter()
    warm_runs = 0
    if warmup > 0:
        plan.execute(warmup)
        warm_runs += warmup
    plan.sync()
    while time.perf_counter() - tw < WARMUP_MIN_S:
        plan.execute(max(1, warmup))
        warm_runs += max(1, warmup)
        plan.sync()
    warm_ms = (time.perf_counter() - tw) * 1e3
    t0 = time.perf_counter()
    ev_ms = plan.execute(steps)  # HIP events on the executor stream, average per step
    plan.sync()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    log(f"[bench] {wl.name} {steps} steps: {wall_ms:.4f} ms/step wall, {ev_ms:.4f} ms/step events "
        f"(after {warm_runs} warm-up runs, {warm_ms:.0f} ms)")
    plan.release_gpu()
    rotated = rotated_pools(wl, steps) if cfg == 4 else None

    flops = wl.flops
    comp = sum(synth.compulsory_bytes(wl, w) for w in wl.waves)
    gath = sum(gathered_bytes(wl, w) for w in wl.waves)
    value = flops / (wall_ms * 1e-3) / 1e12
    path = rep["waves"][0]["path"]
    kernel_key = path + "_" + wl.name.split("_")[0]
    w0 = wl.waves[0]
    mfma_frac = flops / (ev_ms * 1e-3) / 1e12 / FP16_MFMA_PEAK_TFLOPS
    if cfg in (1, 4):  # substrate and intermediate tensors stay in the caches
        achieved = gath / (ev_ms * 1e-3) / 1e9
        roof = {"bound": "l2", "achieved": round(achieved, 1), "peak": round(L2_PEAK_GBS, 1),
                "unit": "GB/s", "frac": round(achieved / L2_PEAK_GBS, 4),
                "traffic": traffic_from_profiles(kernel_key), "gathered_bytes": gath,
                "algorithmic_hbm_bytes": comp,
                "hbm_frac_of_algorithmic": round(comp / (ev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "kernel_ms": round(ev_ms, 5),
                "note": "gathered bytes (every segment row x tokens) from L2/MALL per kernel time "
                        "against the aggregate L2 read bandwidth"}
    else:
        achieved = comp / (ev_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": traffic_from_profiles(kernel_key), "algorithmic_bytes": comp,
                "kernel_ms": round(ev_ms, 5), "mfma_tflops_frac": round(mfma_frac, 4)}
    out = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": "TFLOP/s",
        "ms_per_step": round(wall_ms, 5),
        "warmup_ms": round(warm_ms, 1),
        "warmup_runs": warm_runs,
        "residency": RESIDENCY[cfg],
        "config": {
            "workload": wl.name,
            "substrate_positions": wl.substrate,
            "batch": wl.tokens,
            "neurons_per_wave": w0.cout,
            "clusters_per_neuron": w0.K,
            "S": w0.S,
            "waves": len(wl.waves),
            "act": w0.act,
            "path": path,
        },
        "hbm_gbs": round(comp / (ev_ms * 1e-3) / 1e9, 1),
        "roofline": roof,
        "_wl": wl,
    }
    if rotated is not None:
        out["rotated_pools"] = rotated
    return out


# What stays in the caches across the timed steps of each configuration (one plan replayed).
RESIDENCY = {
    1: "weights (4 MB), segment tables (0.3 MB) and substrate (8 MB) stay cache-resident "
       "across steps: the plumbing configuration measures the L2/MALL-bound gather",
    2: "weights (8 MB) and segment tables (2 MB) may stay in the 256 MB MALL; the 20.5 GB "
       "substrate, 99 % of the algorithmic bytes, streams from HBM every step",
    3: "weights (268 MB) exceed the 256 MB MALL; substrate rows are re-read by ~2.3 tiles",
    4: "weights (134 MB) and segment tables stay in the 256 MB MALL across steps of one plan; "
       "rotated_pools times 4 copies of the plan in rotation (536 MB)",
}


def rotated_pools(wl, steps: int) -> dict:
    """Config 4 over C4_POOLS separately compiled copies of its plan (own weights, segment
    tables and canvas), one run of each in turn: no copy's weights are in the caches when it
    runs again.  Kernel time per run from HIP events on each plan's stream (the runs are
    launched one at a time, so host waits between them are not counted)."""
    from snntome_amd import synth, wavec

    plans = []
    for _ in range(C4_POOLS):
        p = synth.build_graph(wl, wavec).compile()
        p.init_gpu()
        p.fill_input_uniform(wl.seed)
        plans.append(p)
    tw = time.perf_counter()
    while time.perf_counter() - tw < WARMUP_MIN_S:
        for p in plans:
            p.execute(1)
    ms = []
    for k in range(max(steps, 2 * C4_POOLS)):
        ms.append(plans[k % C4_POOLS].execute(1))
    for p in plans:
        p.release_gpu()
    t = float(np.mean(ms))
    log(f"[bench] {wl.name} over {C4_POOLS} rotated plan copies: {t:.4f} ms/run (events)")
    return {"pools": C4_POOLS, "runs": len(ms), "kernel_ms": round(t, 5),
            "value": round(wl.flops / (t * 1e-3) / 1e12, 4), "unit": "TFLOP/s",
            "gathered_gbs": round(sum(gathered_bytes(wl, w) for w in wl.waves) / (t * 1e-3) / 1e9, 1)}


def bench_llm(steps: int, warmup: int, eager: bool, no_cpu: bool = True) -> dict:
    """Config 5: LLM-shaped decoder, 16 x 512-token prefill + 128 greedy decode steps.  One step =
    prefill of all requests, device-side hand-over (token-shift state, last-token ids), then the
    decode steps as replays of one captured HIP graph (argmax -> embedding chained on the device,
    no host round trip).  The prompt ids (32 KB) are uploaded at the start of every step, since
    the prefill's argmax overwrites the plan's id buffer."""
    from snntome_amd import synth, wavec

    t_start = time.perf_counter()
    spec = synth.LLMSpec()
    wts = synth.llm_weights(spec)
    pre = synth.build_llm_graph(spec, wts, decode=False, wavec_mod=wavec).compile()
    dec = synth.build_llm_graph(spec, wts, decode=True, wavec_mod=wavec).compile()
    pre.init_gpu()
    dec.init_gpu()
    pre.use_graph(not eager)
    dec.use_graph(not eager)
    R, P, D = spec.requests, spec.prompt, spec.decode_steps
    prompt = np.random.default_rng(spec.seed).integers(0, spec.vocab, R * P).astype(np.uint32)
    rep = pre.exec_report()["waves"]
    paths = sorted({w["path"] for w in rep})
    ex_flops = sum(w["flops"] for w in rep)
    log(f"[bench] config5 setup {time.perf_counter() - t_start:.1f}s: {len(pre.cmds)} prefill "
        f"commands ({len(rep)} waves, paths {paths}), executed/effective flops "
        f"{ex_flops / (2 * spec.nnz_per_token * R * P):.3f}; "
        f"{'eager launches' if eager else 'HIP-graph replays'}")

    def one_step():
        ms_p = pre.execute(1)
        synth.llm_handoff(spec, pre, dec)
        ms_d = dec.execute(D)
        return ms_p, ms_d

    pre.set_ids(prompt)
    tw = time.perf_counter()
    warm_steps = 0
    xcd_fallback = False
    while warm_steps < max(1, warmup) or time.perf_counter() - tw < WARMUP_MIN_S:
        pre.set_ids(prompt)
        try:
            one_step()
        except RuntimeError as e:
            # XCD-local split-K meetings that found their chunks on different XCDs (the
            # executor checks after every run): rebuild the decode plan without them.
            if "narrow_local=0" not in str(e) or xcd_fallback:
                raise
            log(f"[bench] {e}; decode plan rebuilt with tuning narrow_local=0")
            wavec.set_tuning("narrow_local", 0)
            dec = synth.build_llm_graph(spec, wts, decode=True, wavec_mod=wavec).compile()
            dec.init_gpu()
            dec.use_graph(not eager)
            wavec.set_tuning("narrow_local", -1)
            xcd_fallback = True
            continue
        warm_steps += 1
        dec.sync()
    pre.sync()
    dec.sync()
    warm_ms = (time.perf_counter() - tw) * 1e3
    t0 = time.perf_counter()
    pms, dms = [], []
    for _ in range(steps):
        pre.set_ids(prompt)  # (prompt ids: host input, re-uploaded; 32 KB)
        a, b = one_step()
        pms.append(a)
        dms.append(b)
    dec.sync()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    prefill_ms, decode_ms = float(np.mean(pms)), float(np.mean(dms))
    f_pre = 2.0 * spec.nnz_per_token * R * P
    f_dec = 2.0 * spec.nnz_per_token * R
    total = f_pre + D * f_dec
    value = total / (wall_ms * 1e-3) / 1e12
    w_bytes = dec.summary["total_w_bytes"]
    dec_gbs = w_bytes / (decode_ms * 1e-3) / 1e9
    pre_tf = f_pre / (prefill_ms * 1e-3) / 1e12
    log(f"[bench] config5 {steps} steps: {wall_ms:.2f} ms/step wall; prefill {prefill_ms:.3f} ms "
        f"({pre_tf:.1f} TFLOP/s), decode {decode_ms:.4f} ms/step ({dec_gbs:.0f} GB/s weights)")
    out = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": "TFLOP/s",
        "ms_per_step": round(wall_ms, 4),
        "config": {
            "workload": "config5_llm_decoder",
            "layers": spec.layers, "d": spec.d, "ffn": spec.ffn, "vocab": spec.vocab,
            "S": spec.S, "clusters_kept": [spec.kept(spec.d), spec.kept(spec.ffn)],
            "tile": spec.tile, "token_shift_rf": spec.rf, "requests": R, "prompt": P,
            "decode_steps": D, "paths": paths, "hip_graphs": not eager,
            "xcd_local_splitk": not xcd_fallback,
        },
        "warmup_ms": round(warm_ms, 1),
        "warmup_runs": warm_steps,
        "prefill_ms": round(prefill_ms, 4),
        "prefill_tflops": round(pre_tf, 2),
        "decode_ms_per_step": round(decode_ms, 5),
        "decode_tokens_per_s": round(R / (decode_ms * 1e-3), 1),
        "decode_weight_gbs": round(dec_gbs, 1),
        "executed_over_effective_flops": round(ex_flops / f_pre, 4),
        "roofline": {
            "bound": "mfma",
            "achieved": round(pre_tf, 2),
            "peak": FP16_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(pre_tf / FP16_MFMA_PEAK_TFLOPS, 4),
            "traffic": traffic_from_profiles("llm_prefill_c5"),
            "kernel_ms": round(prefill_ms, 4),
            "scope": "whole prefill plan (all waves and token ops), effective FLOPs",
        },
        "decode_roofline": {
            "bound": "hbm", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
            "scope": "decode step: executed weight bytes / step time",
        },
    }
    if not no_cpu:
        log("[bench] cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline_llm(spec, wts, R * P)
        log(f"[bench] cpu baseline {out['cpu_baseline']}")
    pre.release_gpu()
    dec.release_gpu()
    return out


def bench_projection(name: str, steps: int, warmup: int, tile: int = 0) -> dict:
    """One projection of layer 0 of the config-5 prefill, alone, at its real shape (16 x 512
    tokens, the same pruned weights and pattern-sorted tiles as in the whole plan, input filled
    on the device): the unit a kernel profile of the prefill's MFMA waves is taken on.  Plain
    plan executions, no HIP graph."""
    from snntome_amd import synth, wavec

    spec = synth.LLMSpec()
    wts = synth.llm_weights(spec)
    if tile:
        spec.tile = tile
    p = wts.head if name == "head" else wts.proj[0][name]
    fan = spec.ffn if name == "dn" else spec.d
    act = {"q": "sigmoid", "k": "silu", "g": "silu"}.get(name)
    T = spec.requests * spec.prompt
    g = wavec.WaveGraph(kv_cache_max_seq=0)
    g.add_input("x", fan, 1, T, is_1d=True)
    g.add_pruned_wave(name, "x", "y", p.starts, spec.S, p.weights, p.bias, tile=spec.tile, act=act)
    g.set_output("y")
    plan = g.compile()
    plan.init_gpu()
    plan.fill_input_uniform(spec.seed)
    rep = plan.exec_report()["waves"]
    if warmup > 0:
        plan.execute(warmup)
    plan.sync()
    ms = plan.execute(steps)
    plan.sync()
    plan.release_gpu()
    eff = 2.0 * p.weights.shape[0] * p.weights.shape[1] * T
    ex = float(sum(w["flops"] for w in rep))
    tf = eff / (ms * 1e-3) / 1e12
    log(f"[bench] projection {name}: {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s effective, "
        f"executed x{ex / eff:.3f}, paths {sorted({w['path'] for w in rep})}")
    return {
        "metric": METRIC, "value": round(tf, 3), "unit": "TFLOP/s", "ms_per_step": round(ms, 5),
        "config": {"workload": "config5_prefill_projection", "projection": f"l0.{name}",
                   "neurons": int(p.weights.shape[0]), "inputs_per_neuron": int(p.weights.shape[1]),
                   "fan_in": fan, "tokens": T, "tile": spec.tile,
                   "paths": sorted({w["path"] for w in rep})},
        "executed_over_effective_flops": round(ex / eff, 4),
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": FP16_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / FP16_MFMA_PEAK_TFLOPS, 4),
                     "traffic": None, "kernel_ms": round(ms, 5),
                     "scope": "one projection alone, effective FLOPs"},
    }


def bench_token64(args):
    """The whitepaper's stand-alone Token64 wave (wavec_k44_f16_forward_token64) at its own
    benchmark shape (whitepaper/sparse_wmma_kernel/tests/benchmark_whitepaper_k44.cpp:141-197):
    Cin = 10,000,000 positions, M = 512 tokens (8 tiles of 64), B = 1024 synapses per cluster row,
    Cout = 8192, cluster size S (--cluster).  Index rows uniform over the substrate; weights and
    index rows rotate through a pool of >= 1 GiB (as the reference's ring benchmark does) so that
    every launch streams them from HBM.  TSyn/s = Cout * B * M / t; TFLOP/s = 2 * TSyn/s."""
    from snntome_amd import wavec

    lib = wavec.get_lib()
    Cin, M, B, Cout, S = args.t64_cin, 512, 1024, 8192, args.cluster
    tiles = M // 64
    rng = np.random.default_rng(44)
    log(f"[bench] token64: Cin={Cin:,} M={M} B={B} Cout={Cout} S={S}; filling "
        f"{tiles * Cin * 128 / 1e9:.2f} GB substrate")
    X = wavec.DeviceBuffer(tiles * Cin * 64 * 2)
    if lib.wavec_dev_fill_uniform(X.ptr, tiles * Cin, 64, 64, 0, 7) != 0:
        raise RuntimeError(wavec.last_error())
    w_bytes = Cout * B * 2
    idx_bytes = (Cout // S) * B * 4
    n_sets = max(4, -(-(1 << 30) // (w_bytes + idx_bytes)))
    W = wavec.DeviceBuffer(n_sets * w_bytes)
    I = wavec.DeviceBuffer(n_sets * idx_bytes)
    w0 = wavec.DeviceBuffer.from_array(
        (rng.standard_normal((Cout, B), dtype=np.float32) * 0.02).astype(np.float16))
    for k in range(n_sets):  # distinct index rows per set, same weights (bytes are what matter)
        idx = rng.integers(0, Cin, size=(Cout // S, B), dtype=np.int64).astype(np.uint32)
        lib.wavec_dev_upload(I.ptr + k * idx_bytes, idx.ctypes.data, idx_bytes)
        wavec.interleave_weights_wmma(W.ptr + k * w_bytes, w0, Cout, B // 8)  # WMMA order
    wavec.device_synchronize()
    bias = wavec.DeviceBuffer.from_array(np.zeros(Cout, np.float16))
    Y = wavec.DeviceBuffer(tiles * Cout * 64 * 2)

    def launch(k):
        wavec.forward_token64_f16(Y, X, I.ptr + (k % n_sets) * idx_bytes,
                                  W.ptr + (k % n_sets) * w_bytes, bias, M, Cin, Cout, B // 16, S)

    tw = time.perf_counter()
    warm = 0
    while warm < args.warmup or time.perf_counter() - tw < WARMUP_MIN_S:
        for _ in range(max(1, args.warmup)):
            launch(warm)
            warm += 1
        wavec.device_synchronize()
    warm_ms = (time.perf_counter() - tw) * 1e3
    ms = __import__("ctypes").c_float()
    lib.wavec_dev_time_begin()
    for k in range(args.steps):
        launch(warm + k)
    lib.wavec_dev_time_end(__import__("ctypes").byref(ms))
    t = ms.value * 1e-3 / args.steps
    tsyn = Cout * B * M / t / 1e12
    log(f"[bench] token64 S={S}: {t * 1e6:.1f} us/launch, {tsyn:.2f} TSyn/s, {2 * tsyn:.1f} TFLOP/s")
    out = {
        "metric": METRIC,
        "value": round(2 * tsyn, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_launches": warm, "warmup_ms": round(warm_ms, 1),
        "ms_per_step": round(t * 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16 (fp32 accumulate)",
        "data": "synthetic (device-generated substrate, uniform index rows, N(0,0.02) weights)",
        "config": {"workload": "whitepaper_token64", "Cin": Cin, "M": M, "B": B, "Cout": Cout,
                   "cluster": S, "pool_sets": n_sets},
        "tsyn_per_s": round(tsyn, 3),
    }
    print(json.dumps(out), flush=True)


def bench_conv(args):
    """Dense convolutions of reference-compiled plans whose rows sit off the 16-byte grid: a
    token-shifted 1-D convolution (kw 3 over 512 channels, 4,096 tokens, after a 1x1 so its
    input is not at canvas offset 0) and single-frame 3x3 / 1x1 image convolutions (batch 1,
    128 x 128 padded planes, tiles and taps at any element offset).  Each plan is timed on the
    MFMA tile kernel (rows shifted into place) and with every wave forced to the VALU gathers
    (tuning switch path=0); HIP events on the executor stream, >= 200 ms of warm-up."""
    from snntome_amd import wavec

    rng = np.random.default_rng(31)

    def f16(shape, s):
        return (rng.standard_normal(shape) * s).astype(np.float32)

    def conv1d():
        cin, W = 512, 4096
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("x", cin, 1, W, is_1d=True)
        g.add_linear("pre", "x", "h", cin, cin, f16((cin, cin), 0.04), f16((cin,), 0.05),
                     act="relu")
        g.add_conv2d("conv", "h", "y", cin, cin, 1, 3, f16((cin, cin, 1, 3), 0.03),
                     f16((cin,), 0.05), stride=1, pad=1, act="silu")
        return g, 2.0 * cin * cin * W * (1 + 3)

    def conv2d(k, c, H, W):
        g = wavec.WaveGraph(kv_cache_max_seq=0)
        g.add_input("img", c, H, W)
        g.add_conv2d("conv", "img", "y", c, c, k, k, f16((c, c, k, k), 0.2 / (c * k * k) ** 0.5),
                     f16((c,), 0.05), stride=1, pad=k // 2, act="relu")
        return g, 2.0 * c * c * k * k * H * W

    def fill(plan):
        """Random fp16 input: 1-D plans from the device generator; an image's interior pixels
        through the padded-plane layout (reference K44ResDesc::init: W_pad = W + 8 for widths
        that are multiples of 64, else W + 4; pixel (y, x) of channel c at
        c * channel_stride + (y + 1) * W_pad + 4 + x), halos left zero."""
        c0 = plan.cmds[0]
        if int(c0["h_out"]) <= 1:  # a 1-D token input
            plan.fill_input_uniform(7)
            return
        C, H, W = int(c0["Cin"]), int(c0["h_out"]), int(c0["w_out"])
        aligned = W % 64 == 0
        wp = W + 8 if aligned else W + 4
        ss = (H + 2) * wp if aligned else (2 * wp + (H * wp + 63) // 64 * 64 + 63) & ~63
        off = (np.arange(C)[:, None, None] * ss + (np.arange(H)[None, :, None] + 1) * wp + 4
               + np.arange(W)[None, None, :])
        buf = np.zeros(C * ss, np.float16)
        buf[off.ravel()] = rng.standard_normal(off.size).astype(np.float16)
        plan.write_canvas(int(c0["src_off"]), buf)

    cases = {"conv1d_k3_512ch_4096tok (1x1 + kw3)": conv1d,
             "conv2d_3x3_64ch_128x128_batch1": lambda: conv2d(3, 64, 128, 128),
             "conv2d_1x1_256ch_128x128_batch1": lambda: conv2d(1, 256, 128, 128)}
    out = {}
    for name, make in cases.items():
        rec = {}
        for mode, path in (("mfma", -1), ("valu", 0)):
            wavec.reset_tuning()
            wavec.set_tuning("path", path)
            g, flops = make()
            plan = g.compile()
            plan.init_gpu()
            fill(plan)
            paths = [w["path"] for w in plan.exec_report()["waves"]]
            tw = time.perf_counter()
            while time.perf_counter() - tw < WARMUP_MIN_S:
                plan.execute(max(1, args.warmup))
            ms = plan.execute(args.steps)
            plan.release_gpu()
            rec[mode] = {"ms_per_plan": round(ms, 5), "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                         "paths": paths}
            log(f"[bench] {name} {mode}: {ms:.4f} ms/plan, {flops / (ms * 1e-3) / 1e12:.1f} "
                f"TFLOP/s, waves {paths}")
        rec["flops"] = flops
        rec["mfma_over_valu"] = round(rec["valu"]["ms_per_plan"] / rec["mfma"]["ms_per_plan"], 2)
        out[name] = rec
    wavec.reset_tuning()
    first = next(iter(out.values()))
    print(json.dumps({
        "metric": METRIC, "value": first["mfma"]["tflops"], "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": first["mfma"]["ms_per_plan"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 (fp32 accumulate)",
        "data": "synthetic (device-generated substrate, normal weights)",
        "config": {"workload": "misaligned_dense_convolutions"}, "cases": out}), flush=True)


def _envelope(rec: dict, args, data: str) -> dict:
    """The driver's contract fields around one configuration record."""
    out = {
        "metric": rec["metric"], "value": rec["value"], "unit": rec["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": rec["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 (fp32 accumulate)", "data": data,
    }
    out.update({k: v for k, v in rec.items() if k not in out and not k.startswith("_")})
    if getattr(args, "tune", None):
        out["tuning"] = {kv.partition("=")[0]: int(kv.partition("=")[2]) for kv in args.tune}
    return out


WAVE_DATA = "synthetic (device-generated counter-hash substrate; numpy PCG64 weights)"
LLM_DATA = "synthetic (random-init fp16 weights, uniform random prompt ids)"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=None, choices=[1, 2, 3, 4, 5],
                    help="one configuration alone (default: headline config 2 + all others)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="config 5: launch kernel by kernel (the default; kept for scripts)")
    ap.add_argument("--graphs", action="store_true",
                    help="config 5: replay captured HIP graphs instead of launching kernel by "
                         "kernel (measured 0.8 %% slower on decode: 0.7657 against 0.7595 ms/step)")
    ap.add_argument("--conv", action="store_true",
                    help="dense convolutions with rows off the 16-byte grid, MFMA vs VALU")
    ap.add_argument("--token64", action="store_true",
                    help="the whitepaper's stand-alone Token64 wave at its benchmark shape")
    ap.add_argument("--cluster", type=int, default=128, help="--token64: cluster size S")
    ap.add_argument("--t64-cin", type=int, default=10_000_000, help="--token64: Cin")
    ap.add_argument("--c5-projection", default=None,
                    choices=["q", "k", "v", "o", "g", "u", "dn", "head"],
                    help="one config-5 prefill projection (layer 0) alone, for kernel profiles")
    ap.add_argument("--c5-tile", type=int, default=0,
                    help="--c5-projection: neurons per pattern-sorted tile (default: the spec's)")
    ap.add_argument("--tune", action="append", default=[], metavar="KEY=VALUE",
                    help="executor tuning switch (wavec_set_tuning) for every plan; repeatable")
    ap.add_argument("--copy-probe-gib", type=float, default=0.0,
                    help="only run a plain device copy of this many GiB (PMC calibration)")
    args = ap.parse_args()
    if args.copy_probe_gib > 0:
        copy_probe(args.copy_probe_gib)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(a wave shards by batch columns across GPUs with no communication; this build "
              "runs and measures the one-GPU share)",
              file=sys.stderr)
        sys.exit(2)
    if args.token64:
        bench_token64(args)
        return
    if args.conv:
        bench_conv(args)
        return
    if args.tune:
        from snntome_amd import wavec
        for kv in args.tune:
            key, _, val = kv.partition("=")
            wavec.set_tuning(key, int(val))
    if args.c5_projection:
        rec = bench_projection(args.c5_projection, args.steps, args.warmup, args.c5_tile)
        print(json.dumps(_envelope(rec, args, LLM_DATA)), flush=True)
        return
    # Under rocprofv3 config 5 launches kernel by kernel: a kernel-trace run of its HIP-graph
    # capture ended in a host segmentation fault inside the profiler's preloaded libraries.
    # Kernel-by-kernel launches are the default: alternated in one process, decode steps took
    # 0.7595 ms launched one by one against 0.7657 ms as graph replays (prefill alike).
    eager = args.eager or not args.graphs or under_profiler()
    # Config 5's two-plan workload (alone or in the default run) is not run under counter
    # collection: one such run ended in a host segmentation fault in a thread of the profiling
    # runtime reading a device address, cause unknown.  Counters of config 5 are taken per
    # projection (--c5-projection), configs 1-4 with --config N.
    if (args.config in (None, 5)) and under_counter_collection():
        print("bench.py: config 5 (alone or in the default run) is not run under rocprofv3 "
              "counter collection; take its counters with --c5-projection NAME, and those of "
              "configs 1-4 with --config N", file=sys.stderr)
        sys.exit(3)

    if args.config == 5:
        rec = bench_llm(args.steps, args.warmup, eager, no_cpu=args.no_cpu)
        print(json.dumps(_envelope(rec, args, LLM_DATA)), flush=True)
        return
    if args.config is not None:
        rec = bench_wave(args.config, args.steps, args.warmup)
        out = _envelope(rec, args, WAVE_DATA)
        if not args.no_cpu:
            log("[bench] cpu baseline ...")
            out["cpu_baseline"] = cpu_baseline(rec["_wl"])
        print(json.dumps(out), flush=True)
        return

    # Default: the headline (config 2) plus every other configuration at its full size.
    head = bench_wave(2, args.steps, args.warmup)
    out = _envelope(head, args, WAVE_DATA)
    configs = {}
    for cfg in (1, 3, 4):
        rec = bench_wave(cfg, args.steps, args.warmup)
        configs[f"c{cfg}"] = {k: v for k, v in rec.items() if not k.startswith("_") and k != "metric"}
    rec = bench_llm(1, 1, eager)
    configs["c5"] = {k: v for k, v in rec.items() if k != "metric"}
    configs["c5"]["steps"], configs["c5"]["warmup"] = 1, 1
    out["configs"] = configs
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(head["_wl"])
        log(f"[bench] cpu baseline {out['cpu_baseline']}")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
