#!/usr/bin/env python3
"""MoE-layer throughput on one MI355X (gfx950).

Workload (default, `--workload decode`): the Qwen3.6-35B-A3B-shaped MoE layer
(hidden 2048, 256 experts, top-8 + 1 shared expert, ffn 512, SwiGLU, Q4_0
expert weights from N(0,0.02), f32 router N(0,0.02)) at decode batch 10
(10 tokens, f32 activations N(0,1)).  A step is one layer forward over one
batch.  Steps rotate over `--layers` distinct synthetic layers (8 x 0.87 GB by
default, far above the 256 MB Infinity Cache, so weights stream from HBM) and
`--batches` distinct input batches, so expert sets change from step to step.

Output: ONE JSON line with value = tokens/s of the layer, the HBM roofline of
the dominant kernel (gate/up expert GEMV; per-launch duration from HIP events
recorded by the library on its own stream) and the CPU oracle timed on the
host cores over a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
MFMA_I8_PEAK_TOPS = 5000.0


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
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--workload", default="decode", choices=["decode"])
    ap.add_argument("--tokens", type=int, default=10)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--batches", type=int, default=16)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of HIP graph replays")
    ap.add_argument("--profile-steps", type=int, default=256)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-threads", type=int, default=0, help="0: min(16, os.cpu_count())")
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


def main() -> int:
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the MoE layer on one MI355X); "
              f"--gpus {args.gpus} is not supported.  Expert-parallel sharding is described in DESIGN.md.",
              file=sys.stderr, flush=True)
        return 2

    import numpy as np
    import torch

    from qwenium_amd import Workspace, lib, synthetic
    from qwenium_amd._lib import check, row_bytes

    spec = synthetic.QWEN35B
    T = args.tokens
    H, E, K, F = spec.n_embd, spec.n_experts, spec.top_k, spec.ffn_dim
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    log(f"generating {args.layers} layers ({spec.wtype=}) and {args.batches} input batches on the GPU")
    layers, tensors = [], []
    for l in range(args.layers):
        t = synthetic.make_layer_tensors(spec, args.seed, layer=l, device=dev)
        tensors.append(t)
        layers.append(synthetic.make_layer(spec, args.seed, layer=l, tensors=t))
    xs = [synthetic.make_x(spec, T, args.seed, batch=b, device=dev) for b in range(args.batches)]
    ws = Workspace(layers[0], T)
    y = torch.empty((T, H), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    # schedule: step s uses layer s % L and batch s % B; a graph holds one period
    L, B = args.layers, args.batches
    period = int(np.lcm(L, B))
    sched = [(s % L, s % B) for s in range(period)]

    # routing statistics per (layer, batch): distinct routed experts hit
    distinct = {}
    for (l, b) in sched:
        _, dbg = layers[l].forward(xs[b], out=y, workspace=ws, debug=True)
        distinct[(l, b)] = int(torch.unique(dbg["topk_idx"]).numel())
    torch.cuda.synchronize()
    D_mean = float(np.mean([distinct[p] for p in sched]))

    rb_h = row_bytes(spec.wtype, H)
    rb_f = row_bytes(spec.wtype, F)
    expert_bytes = 2 * F * rb_h + H * rb_f                # gate + up + down of one expert
    shared_bytes = expert_bytes if spec.shared else 0
    router_bytes = E * H * 4 + (H * 4 if spec.shared else 0)
    act_bytes = 2 * T * H * 4                             # x in, y out (f32)
    layer_bytes = D_mean * expert_bytes + shared_bytes + router_bytes + act_bytes
    R = T * K + (T if spec.shared else 0)
    gu_bytes = (D_mean + (1 if spec.shared else 0)) * 2 * F * rb_h + T * (H + H // 32 * 8) + R * (F + F // 32 * 8)

    def run_step(i):
        l, b = sched[i % period]
        layers[l].forward(xs[b], out=y, workspace=ws)

    log(f"warmup {args.warmup} steps")
    for i in range(args.warmup):
        run_step(i)
    torch.cuda.synchronize()

    steps = args.steps
    graph = None
    if not args.eager:
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(period):
                run_step(i)
        for _ in range(2):
            graph.replay()
        torch.cuda.synchronize()
        steps = max(period, (steps // period) * period)

    log(f"timing {steps} steps ({'eager' if args.eager else f'graph of {period} steps'})")
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    if graph is not None:
        for _ in range(steps // period):
            graph.replay()
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

    # per-phase timing on the library's stream: eager steps queued behind a
    # bounded sleep kernel so host launch latency never shows up as GPU time
    log(f"profiling {args.profile_steps} steps with phase events")
    n_ev = 5
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    evs = []
    for _ in range(args.profile_steps * n_ev):
        e = ctypes.c_void_p()
        if hip.hipEventCreate(ctypes.byref(e)) != 0:
            raise RuntimeError("hipEventCreate failed")
        evs.append(e)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2.4e9 * 0.05))  # ~50 ms at 2.4 GHz
    for i in range(args.profile_steps):
        l, b = sched[i % period]
        arr = (ctypes.c_void_p * n_ev)(*[evs[i * n_ev + j].value for j in range(n_ev)])
        check(lib().qmoe_layer_set_phase_events(layers[l]._handle, arr))
        layers[l].forward(xs[b], out=y, workspace=ws)
        check(lib().qmoe_layer_set_phase_events(layers[l]._handle, None))
    torch.cuda.synchronize()
    phase = np.zeros((args.profile_steps, n_ev - 1))
    ms = ctypes.c_float()
    for i in range(args.profile_steps):
        for j in range(n_ev - 1):
            if hip.hipEventElapsedTime(ctypes.byref(ms), evs[i * n_ev + j], evs[i * n_ev + j + 1]) != 0:
                raise RuntimeError("hipEventElapsedTime failed")
            phase[i, j] = ms.value * 1e3
    for e in evs:
        hip.hipEventDestroy(e)
    phase_us = phase.mean(axis=0)
    D_prof = float(np.mean([distinct[sched[i % period]] for i in range(args.profile_steps)]))
    gu_bytes_prof = (D_prof + 1) * 2 * F * rb_h + T * (H + H // 32 * 8) + R * (F + F // 32 * 8)
    gu_us = float(phase_us[1])
    achieved = gu_bytes_prof / (gu_us * 1e-6) / 1e9
    log("phase us: route %.2f gate/up %.2f down %.2f combine %.2f" % tuple(phase_us))

    # parity of one step against the CPU oracle, and the CPU baseline
    result_parity = None
    cpu = None
    if not args.no_cpu:
        from oracle import pyoracle as po

        host = {k: v.data.cpu().numpy() for k, v in tensors[0].items()}
        host["router"] = host["router"].reshape(E, H)
        ref = po.Layer(H, E, K, F, spec.shared, spec.wtype, host)
        x0 = xs[0].cpu().numpy()
        y_gpu, dbg = layers[0].forward(xs[0], workspace=ws, debug=True)
        torch.cuda.synchronize()
        y_ref, d_ref = ref.forward(x0, debug=True)
        y_gpu = y_gpu.cpu().numpy()
        rms = float(np.sqrt(np.mean(y_ref.astype(np.float64) ** 2)))
        result_parity = {
            "routing_bit_exact": bool(np.array_equal(dbg["topk_idx"].cpu().numpy(), d_ref["topk_idx"])
                                      and np.array_equal(dbg["rows"].cpu().numpy(), d_ref["rows"])),
            "max_abs_err_over_rms": float(np.max(np.abs(y_gpu - y_ref)) / rms),
            "bit_identical_frac": float(np.mean(y_gpu.view(np.int32) == y_ref.view(np.int32))),
        }
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        ref.forward(x0, nthreads=threads)  # warm
        iters, t_cpu = 0, 0.0
        t_start = time.perf_counter()
        while t_cpu < args.cpu_seconds:
            ref.forward(x0, nthreads=threads)
            iters += 1
            t_cpu = time.perf_counter() - t_start
        cpu = {
            "value": iters * T / t_cpu,
            "unit": "tokens/s",
            "cores": threads,
            "kind": "port",
            "sample": f"{iters} forwards of layer 0 on decode batch 0 ({T} tokens) in {t_cpu:.1f}s; "
                      f"ggml-semantics CPU restatement (oracle/liboracle.so, OpenMP) on {cpu_model()}",
        }
        log(f"cpu baseline {cpu['value']:.4g} tok/s on {threads} threads")

    out = {
        "metric": "MoE-layer tokens/s at 35B-A3B shape (decode batch 10, Q4_0)",
        "value": tok_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8_0 int8 dot, f64-exact accumulation, f32 activations",
        "data": "synthetic (seeded, generated on device; random-init weights of the 35B-A3B MoE layer shape)",
        "config": {
            "workload": f"Qwen3.6-35B-A3B MoE layer, decode batch {T}: hidden {H}, {E} experts, top-{K} + shared, "
                        f"ffn {F}, Q4_0",
            "tokens": T, "hidden": H, "experts": E, "top_k": K, "ffn": F, "shared_expert": spec.shared,
            "weight_type": "Q4_0", "distinct_layers": L, "distinct_batches": B, "timing": "eager" if args.eager
            else f"hip graph of {period} steps",
        },
        "layer_hbm": {
            "distinct_experts_mean": D_mean,
            "algorithmic_bytes_per_step": layer_bytes,
            "achieved_GBs": layer_bytes / (ms_per_step * 1e-3) / 1e9,
            "frac_of_peak": layer_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        },
        "phase_us": {"route": phase_us[0], "gate_up": phase_us[1], "down": phase_us[2], "combine": phase_us[3]},
        "roofline": {
            "bound": "hbm",
            "kernel": "k_gateup_gemv (gate+up expert GEMV, SwiGLU, Q8_0 epilogue)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None,
            "bytes_per_launch": gu_bytes_prof,
            "avg_launch_us": gu_us,
        },
        "cpu_baseline": cpu,
        "parity": result_parity,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
