#!/usr/bin/env python3
"""MoE-layer throughput on one MI355X (gfx950).

Workloads (Qwen3.6-35B-A3B MoE layer shape: hidden 2048, 256 experts, top-8 +
1 shared expert, ffn 512, SwiGLU; synthetic seeded weights N(0,0.02) in GGUF
block layout, f32 router N(0,0.02), f32 activations N(0,1)):

  decode             10 tokens, Q4_0 experts.  HBM-bound.  Steps rotate over
                     --layers distinct layers (8 x 0.45 GB by default, far above
                     the 256 MB Infinity Cache) and --batches input batches.
  prefill            4096 tokens, Q4_0 experts.  f16-MFMA path (exact block dots).
  skewed             2048 tokens, Q8_0 experts, Zipf(1.2)-skewed routing: ~50% of
                     assignments on 8 hot experts, ~46 experts empty.
  stack              40 consecutive layers, each x <- x + MoE(RMSNorm(x) * w):
                     --tokens 1 / 10 (default) / 64 (decode) or 8192 (prefill).
  gemma4-decode      Gemma 4 26B-A4B GeGLU MoE layer (hidden 2816, 128 experts,
  gemma4-prefill     top-8, ffn 704, fused gate_up, no shared expert), 10 / 4096
                     tokens, Q4_0; a step is build_moe_geglu(expert_in, router_in)
                     on inputs prepared from the residual rows beforehand.

Without --workload the run is the decode line (the headline: value, roofline,
cpu_baseline) with the 4096-token prefill measured in the same process under
"prefill" (its own MFMA roofline and CPU baseline).  A step is one layer
forward over one batch (stack: one pass over all 40 layers); exactly --steps
steps are timed.  The roofline's per-launch duration comes from HIP events the
library records around the dominant kernel on its own stream; HBM traffic per
launch from the committed rocprofv3 counter summary, when one exists.  The CPU
oracle is timed on the host cores over a bounded sample: the median of >= 10
forwards after 3 warm-ups, on all cores of the process's share and on 4
threads (ggml's default thread count).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
MFMA_I8_PEAK_TOPS = 5000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16 MFMA (the instruction the prefill GEMMs run)

WORKLOADS = {
    # name: (tokens, layer spec name, default layers, default batches, default steps, warmup)
    "decode": (10, "QWEN35B", 8, 16, 2000, 64),
    "prefill": (4096, "QWEN35B", 4, 2, 64, 8),
    "skewed": (2048, "QWEN35B_SKEW", 4, 2, 64, 8),
    "stack": (10, "QWEN35B", 40, 2, 32, 4),
    "gemma4-decode": (10, "GEMMA4", 8, 16, 2000, 64),
    "gemma4-prefill": (4096, "GEMMA4", 4, 2, 64, 8),
}
STACK_LAYERS = 40
CPU_MIN_FORWARDS = 10
CPU_WARMUP = 3
GGML_DEFAULT_THREADS = 4


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", default=None, choices=sorted(WORKLOADS),
                    help="one workload only (default: decode, plus the prefill leg)")
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--batches", type=int, default=None)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of HIP graph replays")
    ap.add_argument("--profile-steps", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="per CPU leg: keep timing forwards (beyond the first 10) until this much time has passed")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0: min(16, os.cpu_count())")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after the run, copy this many MiB device-to-device 4 times (calibration dispatches "
                         "for HBM traffic counters)")
    return ap.parse_args()


class PhaseEvents:
    """Per-step HIP events recorded by the library around its phases."""

    N = 5

    def __init__(self, n_steps: int):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.evs = []
        for _ in range(n_steps * self.N):
            e = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.evs.append(e)

    def arr(self, step: int):
        return (ctypes.c_void_p * self.N)(*[self.evs[step * self.N + j].value for j in range(self.N)])

    def phases_us(self, n_steps: int):
        import numpy as np
        out = np.zeros((n_steps, self.N - 1))
        ms = ctypes.c_float()
        for i in range(n_steps):
            for j in range(self.N - 1):
                if self.hip.hipEventElapsedTime(ctypes.byref(ms), self.evs[i * self.N + j],
                                                self.evs[i * self.N + j + 1]) != 0:
                    raise RuntimeError("hipEventElapsedTime failed")
                out[i, j] = ms.value * 1e3
        return out

    def close(self):
        for e in self.evs:
            self.hip.hipEventDestroy(e)


class LayerPool:
    """Synthetic layers generated on the GPU once and shared by the legs of a run."""

    def __init__(self, seed: int, dev):
        self.seed, self.dev = seed, dev
        self.cache = {}

    def get(self, spec_name: str, n: int, norms: bool = False):
        from qwenium_amd import synthetic

        spec = getattr(synthetic, spec_name)
        have = self.cache.setdefault(spec_name, {"layers": [], "tensors": [], "norms": []})
        while len(have["layers"]) < n:
            l = len(have["layers"])
            t = synthetic.make_layer_tensors(spec, self.seed, layer=l, device=self.dev)
            have["tensors"].append(t)
            have["layers"].append(synthetic.make_layer(spec, self.seed, layer=l, tensors=t))
        while norms and len(have["norms"]) < n:
            have["norms"].append(synthetic.make_norm_weight(spec, self.seed, len(have["norms"]), device=self.dev))
        return spec, have["layers"][:n], have["tensors"][:n], have["norms"][:n]


def cpu_legs(run, n_tok: int, threads_all: int, seconds: float, divide: int = 1) -> dict:
    """Median tokens/s of the CPU oracle over >= CPU_MIN_FORWARDS forwards after
    CPU_WARMUP warm-ups, on all threads of the share and on ggml's default 4."""
    import numpy as np

    legs = []
    for threads in sorted({threads_all, GGML_DEFAULT_THREADS}, reverse=True):
        for _ in range(CPU_WARMUP):
            run(threads)
        times = []
        t_start = time.perf_counter()
        while len(times) < CPU_MIN_FORWARDS or (time.perf_counter() - t_start < seconds and len(times) < 200):
            t0 = time.perf_counter()
            run(threads)
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        legs.append({"threads": threads, "forwards": len(times), "median_s": med,
                     "tok_per_s": n_tok / med / divide})
        log(f"cpu leg: {threads} threads, median {med * 1e3:.1f} ms per forward of {n_tok} tokens "
            f"-> {n_tok / med / divide:.4g} tok/s")
    return {leg["threads"]: leg for leg in legs}


def run_leg(args, pool: LayerPool, workload: str, headline: bool) -> dict:
    import numpy as np
    import torch

    from qwenium_amd import TYPE_Q4_0, Workspace, gemma4_moe_inputs, lib, rms_norm, ssq_parts, synthetic
    from qwenium_amd._lib import check, row_bytes

    T0, spec_name, L0, B0, S0, W0 = WORKLOADS[workload]
    stack = workload == "stack"
    # --tokens / --layers / --batches shape the selected workload only
    T = (args.tokens if headline and args.tokens else None) or T0
    L = STACK_LAYERS if stack else ((args.layers if headline and args.layers else None) or L0)
    B = (args.batches if headline and args.batches else None) or B0
    steps = args.steps or S0
    warmup = args.warmup if args.warmup is not None else W0
    dev = pool.dev
    log(f"workload {workload}: T={T}, {L} layers, {B} input batches (generated on the GPU)")
    spec, layers, tensors, norms = pool.get(spec_name, L, norms=stack)
    H, E, K, F = spec.n_embd, spec.n_experts, spec.top_k, spec.ffn_dim
    wname = "Q4_0" if spec.wtype == TYPE_Q4_0 else "Q8_0"
    xs = [synthetic.make_x(spec, T, args.seed, batch=b, device=dev) for b in range(B)]
    geglu = spec.geglu
    if geglu:
        # build_moe_geglu's two inputs per batch (gemma4.cpp:555-563), prepared outside the timed steps
        g4_norms = synthetic.make_gemma4_norms(spec, args.seed, 0, device=dev)
        g4_in = [gemma4_moe_inputs(x, *g4_norms, synthetic.NORM_EPS) for x in xs]
    ws = Workspace(layers[0], T)
    y = torch.empty((T, H), dtype=torch.float32, device=dev)
    hbuf = torch.empty((T, H), dtype=torch.float32, device=dev)
    xbuf = [torch.empty((T, H), dtype=torch.float32, device=dev) for _ in range(2)]
    # at decode sizes each block's RMSNorm partial sums go to the next block (its
    # routing then finishes the sum instead of reading x for it)
    carry = stack and T <= 16
    sbuf = [torch.empty((T, ssq_parts(H)), dtype=torch.float64, device=dev) for _ in range(2)] if carry else None
    torch.cuda.synchronize()

    def stack_pass(b, keep=None):
        """x <- x + MoE_l(RMSNorm(x) * w_l) for l = 0..L-1 (qwen36.cpp:297-304); keep[l] gets layer l's input."""
        cur, cur_ssq = xs[b], None
        for l in range(L):
            if keep is not None and l in keep:
                keep[l] = cur.clone()
            nxt = xbuf[l & 1]
            nxt_ssq = sbuf[l & 1] if carry else None
            # the block's slice in one call: nxt = cur + MoE(RMSNorm(cur) * w_l)
            layers[l].forward_norm(cur, norms[l], synthetic.NORM_EPS, out=nxt, workspace=ws, x_ssq=cur_ssq,
                                   y_ssq=nxt_ssq)
            cur, cur_ssq = nxt, nxt_ssq
        return cur

    if stack:
        period = B
        sched = [(None, s % B) for s in range(period)]
    else:
        period = int(np.lcm(L, B))
        sched = [(s % L, s % B) for s in range(period)]

    def layer_forward(l, b, **kw):
        if geglu:
            return layers[l].forward_routed(g4_in[b][0], g4_in[b][1], out=y, workspace=ws, **kw)
        return layers[l].forward(xs[b], out=y, workspace=ws, **kw)

    def run_step(i):
        l, b = sched[i % period]
        if stack:
            stack_pass(b)
        else:
            layer_forward(l, b)

    # routing statistics: distinct routed experts hit per (layer, batch) forward
    distinct = []
    if stack:
        cur = xs[0]
        for l in range(L):
            rms_norm(cur, norms[l], synthetic.NORM_EPS, out=hbuf)
            _, dbg = layers[l].forward(hbuf, out=xbuf[l & 1], workspace=ws, residual=cur, debug=True)
            distinct.append(int(torch.unique(dbg["topk_idx"]).numel()))
            cur = xbuf[l & 1]
    else:
        for (l, b) in sched:
            _, dbg = layer_forward(l, b, debug=True)
            distinct.append(int(torch.unique(dbg["topk_idx"]).numel()))
    torch.cuda.synchronize()
    D_mean = float(np.mean(distinct))
    skew_stats = None
    if spec.skew is not None:
        counts = torch.bincount(dbg["topk_idx"].reshape(-1).long(), minlength=E).cpu().numpy()
        hot = spec.skew.hot_experts(E)
        skew_stats = {"hot8_share": float(counts[hot].sum() / counts.sum()), "empty_experts": int((counts == 0).sum()),
                      "max_rows": int(counts.max()), "nonempty_min_rows": int(counts[counts > 0].min())}
        log(f"skew: {skew_stats}")

    rb_h = row_bytes(spec.wtype, H)
    rb_f = row_bytes(spec.wtype, F)
    expert_bytes = 2 * F * rb_h + H * rb_f
    S = 1 if spec.shared else 0
    router_bytes = E * H * 4 + S * H * 4
    R = T * K + S * T
    layer_bytes = (D_mean + S) * expert_bytes + router_bytes + (3 if geglu else 2) * T * H * 4
    ops_gu = 2.0 * R * 2 * F * H      # the GEMMs' multiply-adds x2 (quant x quant), gate + up
    ops_dn = 2.0 * R * H * F
    layer_ops = ops_gu + ops_dn
    mfma_path = T >= 128               # the library's default switch to the grouped f16-MFMA GEMMs

    log(f"warmup {warmup} steps")
    for i in range(warmup):
        run_step(i)
    torch.cuda.synchronize()

    # exactly `steps` steps: whole graphs of `period` steps, then a graph of the remainder
    graphs = []
    if not args.eager:
        stream = torch.cuda.Stream()
        full, rem = steps // period, steps % period
        for n, reps in ((period, full), (rem, 1)):
            if n == 0 or reps == 0:
                continue
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(n):
                    run_step(i)
            graphs.append((g, reps))
        for g, _ in graphs:
            g.replay()
        torch.cuda.synchronize()
    timing = "eager" if args.eager else (
        f"hip graph of {period} steps x {steps // period}" + (f" + graph of {steps % period}" if steps % period else ""))
    log(f"timing {steps} steps ({timing})")
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    if graphs:
        for g, reps in graphs:
            for _ in range(reps):
                g.replay()
    else:
        for i in range(steps):
            run_step(i)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = gpu_ms / steps
    tok_per_s = steps * T / (gpu_ms / 1e3)
    log(f"{ms_per_step * 1e3:.2f} us/step, {tok_per_s:.4g} tok/s (wall {wall:.3f}s)")

    # per-phase timing on the library's stream: eager layer forwards queued behind a
    # bounded sleep kernel so host launch latency never shows up as GPU time
    n_prof = args.profile_steps or (256 if T <= 64 else 16)
    log(f"profiling {n_prof} layer forwards with phase events")
    pe = PhaseEvents(n_prof)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2.4e9 * 0.05))  # ~50 ms at 2.4 GHz
    for i in range(n_prof):
        l, b = (i % L, 0) if stack else sched[i % period]
        check(lib().qmoe_layer_set_phase_events(layers[l]._handle, pe.arr(i)))
        layer_forward(l, b)
        check(lib().qmoe_layer_set_phase_events(layers[l]._handle, None))
    torch.cuda.synchronize()
    phase = pe.phases_us(n_prof)
    pe.close()
    phase_us = phase.mean(axis=0)
    D_prof = D_mean if stack else float(np.mean([distinct[i % period] for i in range(n_prof)]))
    gu_us = float(phase_us[1])
    fused_combine = T <= 16
    if fused_combine:
        # the combine runs in the down kernel: events [3] and [4] are back to back
        phases = {"route": phase_us[0], "gate_up": phase_us[1], "down_combine": phase_us[2] + phase_us[3]}
    else:
        # MFMA path: SwiGLU and the Q8_0 of h run in the gate/up kernel; the exact
        # recomputation of uncertain h values precedes the down kernel
        phases = {"route": phase_us[0], "gate_up": phase_us[1],
                  ("fixup_down" if mfma_path else "hquant_down"): phase_us[2], "combine": phase_us[3]}
    log("phase us: " + ", ".join(f"{k} {v:.2f}" for k, v in phases.items()))

    # HBM traffic per launch of the dominant kernel, measured by rocprofv3 FETCH_SIZE /
    # WRITE_SIZE passes and scaled by a known-size copy (summary committed under profiles/)
    traffic = None
    tpath = os.path.join(REPO, "profiles", f"traffic_{workload}.json")
    if os.path.exists(tpath) and not stack:
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    if not mfma_path:
        if T <= 16:
            # k_gateup_q: routed experts' gate+up rows, the token rows of x (Q8_0), h written as
            # Q8_0 (the shared expert's gate/up runs inside the routing launch); with a shared
            # expert of F = 512, also its down rows, its h rows and the f32 rows ysh it writes
            gu_bytes = D_prof * 2 * F * rb_h + T * (H + H // 32 * 8) + T * K * (F + F // 32 * 8)
            if S and F == 512:
                gu_bytes += H * rb_f + T * (F + F // 32 * 8) + T * H * 4
            gu_kernel = (f"k_gateup_q (routed gate+up expert GEMV with {'GeGLU' if geglu else 'SwiGLU'} and Q8_0 of h, "
                         "one Q8_0 block per workgroup)")
        else:
            gu_bytes = (D_prof + S) * 2 * F * rb_h + T * (H + H // 32 * 8) + R * F * 8
            gu_kernel = "k_gateup_stream (gate+up expert GEMV, prefetching persistent waves)"
        achieved = gu_bytes / (gu_us * 1e-6) / 1e9
        roofline = {
            "bound": "hbm", "kernel": gu_kernel,
            "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic, "bytes_per_launch": gu_bytes, "avg_launch_us": gu_us,
        }
    else:
        achieved = ops_gu / (gu_us * 1e-6) / 1e12
        roofline = {
            "bound": "mfma",
            "kernel": ("k_expert_f16<gate/up> (f16 MFMA grouped GEMM: exact integer block dots and scale "
                       "products, f32 accumulation, SwiGLU and Q8_0 of h in the epilogue)"),
            # priced against the dense int8 peak (the integer block dots' own denominator);
            # the instruction that runs them is the f16 MFMA, whose fraction is beside it
            "achieved": achieved, "peak": MFMA_I8_PEAK_TOPS, "unit": "TFLOP/s",
            "peak_kind": "dense int8 MFMA, 5.0 POP/s (block-dot multiply-adds counted as 2 ops)",
            "frac": achieved / MFMA_I8_PEAK_TOPS, "frac_of_f16_peak": achieved / MFMA_F16_PEAK_TFLOPS,
            "traffic": traffic, "ops_per_launch": ops_gu, "avg_launch_us": gu_us,
        }
    layer_us = ms_per_step * 1e3 / (L if stack else 1)
    layer_rate = {
        "distinct_experts_mean": D_mean, "algorithmic_bytes_per_layer": layer_bytes,
        "hbm_GBs": layer_bytes / (layer_us * 1e-6) / 1e9,
        "frac_of_hbm_peak": layer_bytes / (layer_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "gemm_ops_per_layer": layer_ops,
        "gemm_TOPs": layer_ops / (layer_us * 1e-6) / 1e12,
        "frac_of_f16_mfma_peak": layer_ops / (layer_us * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS,
        "frac_of_int8_mfma_peak": layer_ops / (layer_us * 1e-6) / 1e12 / MFMA_I8_PEAK_TOPS,
        "us_per_layer": layer_us,
    }
    if skew_stats is not None:
        layer_rate["routing"] = skew_stats
    if stack:
        layer_rate["us_per_token"] = ms_per_step * 1e3 / T
    if stack:
        metric = f"MoE-stack tokens/s (40 layers of the 35B-A3B MoE block with RMSNorm, {T} tokens, {wname})"
    elif geglu:
        metric = (f"MoE-layer tokens/s at Gemma 4 26B-A4B shape (GeGLU, "
                  f"{'decode batch' if T <= 64 else 'prefill'} {T}{'' if T <= 64 else ' tokens'}, {wname})")
    elif workload == "decode":
        metric = f"MoE-layer tokens/s at 35B-A3B shape (decode batch {T}, {wname})"
    elif workload == "skewed":
        metric = f"MoE-layer tokens/s at 35B-A3B shape (Zipf-skewed routing, {T} tokens, {wname})"
    else:
        metric = f"MoE-layer tokens/s at 35B-A3B shape (prefill {T} tokens, {wname})"

    # parity against the CPU oracle (stack: layers 0 and L-1 on their actual inputs), and the CPU baseline
    result_parity = None
    cpu = None
    if not args.no_cpu:
        from oracle import pyoracle as po

        def host_layer(l):
            host = {k: v.data.cpu().numpy() for k, v in tensors[l].items()}
            host["router"] = host["router"].reshape(E, H)
            return po.Layer(H, E, K, F, spec.shared, spec.wtype, host,
                            act=po.ACT_GELU_TANH if geglu else po.ACT_SILU)

        n_chk = min(T, 32)
        checks = []
        if stack:
            keep = {0: None, L - 1: None}
            stack_pass(0, keep=keep)
            torch.cuda.synchronize()
            for l in (0, L - 1):
                xin = keep[l]
                rms_norm(xin, norms[l], synthetic.NORM_EPS, out=hbuf)
                yl, dbg = layers[l].forward(hbuf, workspace=ws, residual=xin, debug=True)
                torch.cuda.synchronize()
                hh = po.rms_norm(xin.cpu().numpy()[:n_chk], norms[l].cpu().numpy(), synthetic.NORM_EPS)
                yr, dr = host_layer(l).forward(hh, debug=True)
                yr = yr + xin.cpu().numpy()[:n_chk]
                checks.append((l, yl.cpu().numpy()[:n_chk], yr, dbg["topk_idx"].cpu().numpy()[:n_chk], dr["topk_idx"]))
        elif geglu:
            yl, dbg = layers[0].forward_routed(g4_in[0][0], g4_in[0][1], workspace=ws, debug=True)
            torch.cuda.synchronize()
            yr, dr = host_layer(0).forward(g4_in[0][0].cpu().numpy()[:n_chk], debug=True,
                                           router_in=g4_in[0][1].cpu().numpy()[:n_chk])
            checks.append((0, yl.cpu().numpy()[:n_chk], yr, dbg["topk_idx"].cpu().numpy()[:n_chk], dr["topk_idx"]))
        else:
            yl, dbg = layers[0].forward(xs[0], workspace=ws, debug=True)
            torch.cuda.synchronize()
            yr, dr = host_layer(0).forward(xs[0].cpu().numpy()[:n_chk], debug=True)
            checks.append((0, yl.cpu().numpy()[:n_chk], yr, dbg["topk_idx"].cpu().numpy()[:n_chk], dr["topk_idx"]))
        result_parity = {"tokens_checked": n_chk, "layers_checked": [c[0] for c in checks]}
        for (l, yg, yr, ig, ir) in checks:
            rms = float(np.sqrt(np.mean(yr.astype(np.float64) ** 2)))
            result_parity[f"layer{l}"] = {
                "routing_bit_exact": bool(np.array_equal(ig, ir)),
                "max_abs_err_over_rms": float(np.max(np.abs(yg - yr)) / rms),
                "bit_identical_frac": float(np.mean(yg.view(np.int32) == yr.view(np.int32))),
            }
        threads_all = args.cpu_threads or min(16, os.cpu_count() or 1)
        ref = host_layer(0)
        n_cpu_tok = min(T, 10 if T <= 64 else 256)
        xc = (g4_in[0][0] if geglu else xs[0]).cpu().numpy()[:n_cpu_tok]
        xrc = g4_in[0][1].cpu().numpy()[:n_cpu_tok] if geglu else None
        legs = cpu_legs(lambda th: ref.forward(xc, nthreads=th, router_in=xrc), n_cpu_tok, threads_all,
                        args.cpu_seconds, divide=L if stack else 1)
        main_leg = legs[threads_all]
        cpu = {
            "value": main_leg["tok_per_s"], "unit": "tokens/s", "cores": threads_all, "kind": "port",
            "sample": (f"median of {main_leg['forwards']} forwards (after {CPU_WARMUP} warm-ups) of layer 0 on "
                       f"{n_cpu_tok} tokens of batch 0" + (f", divided by the {L} layers of the stack" if stack else "")
                       + f"; ggml-semantics CPU restatement (oracle/liboracle.so, OpenMP, exact f64 block sums) "
                       f"on {cpu_model()}"),
            "legs": [{"threads": th, "tok_per_s": lg["tok_per_s"], "median_ms_per_forward": lg["median_s"] * 1e3,
                      "forwards": lg["forwards"]} for th, lg in sorted(legs.items())],
        }

    # synchronizes and raises on any device error of the run (no kernel waits on another workgroup)
    if ws.check():
        raise RuntimeError(f"workload {workload}: the workspace check reported a fault")
    return {
        "metric": metric,
        "value": tok_per_s,
        "unit": "tokens/s",
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "dtype": (f"{wname.lower()} x q8_0 block dots on f16 MFMA (exact), f32 accumulation" if mfma_path else
                  f"{wname.lower()} x q8_0 int8 dot (exact), f32 activations"),
        "config": {
            "workload": (f"{L} x Qwen3.6-35B-A3B MoE block (RMSNorm + MoE + residual), {T} tokens" if stack else
                         f"Gemma 4 26B-A4B GeGLU MoE layer, {workload} {T} tokens" if geglu else
                         f"Qwen3.6-35B-A3B MoE layer, {workload} {T} tokens") +
                        f": hidden {H}, {E} experts, top-{K}{' + shared' if spec.shared else ''}, ffn {F}, {wname}" +
                        (f"; {D_mean:.1f} distinct routed experts per forward on average" if T <= 64 else ""),
            "tokens": T, "hidden": H, "experts": E, "top_k": K, "ffn": F, "shared_expert": spec.shared,
            "weight_type": wname, "layers": L, "distinct_batches": B, "timing": timing,
            "prefill_copies": True,
        },
        "layer": layer_rate,
        "phase_us": {"note": "eager forwards with events between phases (event overhead included)", **phases},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity": result_parity,
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the MoE layer on one MI355X); "
              f"--gpus {args.gpus} is not supported: expert-parallel sharding across GPUs is not built.",
              file=sys.stderr, flush=True)
        return 2

    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    pool = LayerPool(args.seed, dev)
    head_name = args.workload or "decode"
    head = run_leg(args, pool, head_name, headline=True)
    extra = {}
    if args.workload is None:
        # the prefill part of the metric, in the same process on the same layers
        extra["prefill"] = run_leg(args, pool, "prefill", headline=False)

    if args.copy_mib > 0:
        n = args.copy_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copies: 4 x {args.copy_mib} MiB device-to-device")
        del src, dst

    out = {
        "metric": head["metric"],
        "value": head["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": head["warmup"],
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": ("synthetic (seeded, generated on device; random-init weights of the "
                 f"{'Gemma 4 26B-A4B' if head_name.startswith('gemma4') else '35B-A3B'} MoE layer shape)"),
        "config": head["config"],
        "layer": head["layer"],
        "phase_us": head["phase_us"],
        "roofline": head["roofline"],
        "cpu_baseline": head["cpu_baseline"],
        "parity": head["parity"],
    }
    out.update(extra)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
