"""Benchmark of the fused quantized MoE expert path on one MI355X.

Workload: the Qwen3-30B-A3B expert decode step -- 48 layers, each with its own
128 resident experts (gate/up 768x2048 q4_K, down 2048x768 q6_K; 18.8 GB of
HBM), top-8 experts per layer drawn from a Zipf(1.1) popularity over a seeded
permutation, router weights softmaxed over the selected 8, batch 1, and the
hidden state carried layer to layer as h <- h + MoE_l(RMSNorm(h)) (eps 1e-6,
tinygiant/engine.py:281-282,335-341).  One step = one token through all 48
expert layers.

Prints one JSON line.  `value` is tokens/s of the device-resident step with
every weight already in HBM (HIP events over K steps); `roofline` is the
dominant kernel's achieved weight bandwidth; `cpu_baseline` is the scalar C
oracle (a restatement of csrc/libtinygiant.c) on this host's cores over a
bounded sample of the same step.
"""

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "expert-FFN tok/s + weight HBM GB/s (% of 8 TB/s), Qwen3-30B-A3B q4_K decode"
HBM_PEAK_GBS = 8000.0
D, I, E, TOPK, L = 2048, 768, 128, 8, 48
GATE_B = I * (D // 256) * 144          # 884,736
DOWN_B = D * (I // 256) * 210          # 1,290,240
EXPERT_B = 2 * GATE_B + DOWN_B         # 3,059,712
SEED = 20261201


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def routing(layers, seed=SEED):
    """Per layer: sorted expert ids and their router weights (top-8 Zipf)."""
    import tinygiant_amd.synth as S
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    out = []
    for _ in range(layers):
        idx = S.zipf_topk(rng, E, TOPK, 1.1, perm)
        w = S.router_weights(rng, TOPK)
        order = np.argsort(idx)
        out.append((idx[order].astype(np.int64), w[order]))
    return out


def setup_gpu(tg, layers, routes):
    """Allocates and fills every layer's 128 experts in HBM; builds the plans."""
    import tinygiant_amd.synth as S
    lib = tg.lib()
    bufs, plans = [], []
    for l in range(layers):
        buf = tg.DeviceArray(E * EXPERT_B)
        base = buf.ptr
        for e in range(E):
            g = base + e * GATE_B
            u = base + E * GATE_B + e * GATE_B
            d = base + 2 * E * GATE_B + e * DOWN_B
            lib.tg_hip_synth_fill(0, S.tensor_seed(SEED, l, e, 0), g, GATE_B, None)
            lib.tg_hip_synth_fill(0, S.tensor_seed(SEED, l, e, 1), u, GATE_B, None)
            lib.tg_hip_synth_fill(2, S.tensor_seed(SEED, l, e, 2), d, DOWN_B, None)
        idx, w = routes[l]
        n = len(idx)
        gp = (ctypes.c_void_p * n)(*[base + int(e) * GATE_B for e in idx])
        up = (ctypes.c_void_p * n)(*[base + E * GATE_B + int(e) * GATE_B for e in idx])
        dp = (ctypes.c_void_p * n)(*[base + 2 * E * GATE_B + int(e) * DOWN_B for e in idx])
        fm = np.full(n, tg.FMT_Q6K, np.int32)
        rw = np.ascontiguousarray(w.reshape(n, 1), dtype=np.float32)
        plan = lib.tg_hip_moe_plan_create(ctypes.addressof(gp), ctypes.addressof(up), ctypes.addressof(dp),
                                          tg.FMT_Q4K, fm.ctypes.data, None, None, None, tg.ACT_SILU, n,
                                          rw.ctypes.data, 1, D, I)
        if not plan:
            raise RuntimeError(tg.last_error())
        bufs.append(buf)
        plans.append(plan)
        if l % 8 == 7:
            log(f"  layers filled: {l + 1}/{layers}")
    lib.tg_hip_synchronize()
    return bufs, plans


def cpu_baseline(routes, sample_layers, min_seconds=10.0, max_reps=400):
    """Oracle (scalar C restatement) over the first `sample_layers` layers of
    the same step: same seeds, same routing, same RMSNorm chain."""
    import oracle
    import tinygiant_amd.synth as S
    try:
        cpus = len(os.sched_getaffinity(0))
    except AttributeError:
        cpus = os.cpu_count() or 2
    threads = max(1, min(16, cpus // 2))
    oracle.set_threads(threads)
    layers = []
    for l in range(sample_layers):
        idx, w = routes[l]
        g = [S.matrix_host(0, S.tensor_seed(SEED, l, int(e), 0), I, D) for e in idx]
        u = [S.matrix_host(0, S.tensor_seed(SEED, l, int(e), 1), I, D) for e in idx]
        d = [S.matrix_host(2, S.tensor_seed(SEED, l, int(e), 2), D, I) for e in idx]
        layers.append((g, u, d, w.reshape(-1, 1).astype(np.float32)))
    ones = np.ones(D, np.float32)
    h = np.random.default_rng(SEED + 1).standard_normal(D).astype(np.float32)
    per_layer = []
    t_total = 0.0
    reps = 0
    while reps < max_reps and (t_total < min_seconds or reps == 0):
        for (g, u, d, w) in layers:
            t0 = time.perf_counter()
            x = oracle.rms_norm(h, ones, 1e-6)
            out = h.reshape(1, D).copy()
            oracle.moe_v2(g, u, d, 0, [2] * len(g), None, None, None, 0, w, x.reshape(1, D), out, I)
            h = out.reshape(D)
            dt = time.perf_counter() - t0
            per_layer.append(dt)
            t_total += dt
        reps += 1
    layer_s = float(np.mean(per_layer))
    step_s = layer_s * L
    return {
        "value": round(1.0 / step_s, 3), "unit": "tok/s", "cores": threads, "kind": "port",
        "sample": (f"{sample_layers} of {L} layers of the same decode step (same seeds and routing), "
                   f"{reps} pass(es), {len(per_layer)} layer calls in {t_total:.1f} s; "
                   f"mean {layer_s * 1e3:.2f} ms/layer scaled x{L}; oracle/tg_oracle.c, gcc -O2, "
                   f"OpenMP over the reference's 96/256-row task split"),
        "weight_gbps": round(TOPK * EXPERT_B / layer_s / 1e9, 2),
    }


def read_traffic():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), if present."""
    p = ROOT / "profiles" / "pmc_moe_gate_up_qwen_decode.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=L)
    ap.add_argument("--cpu-layers", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the expert path is "
              f"built and measured on a single MI355X).", file=sys.stderr)
        return 2

    import tinygiant_amd as tg
    lib = tg.lib()
    name = ctypes.create_string_buffer(256)
    lib.tg_hip_device_name(name, 256)
    log(f"device: {name.value.decode()}")
    layers = args.layers
    routes = routing(layers)
    t0 = time.perf_counter()
    bufs, plans = setup_gpu(tg, layers, routes)
    log(f"resident experts: {layers * E * EXPERT_B / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s")

    h0 = np.random.default_rng(SEED + 1).standard_normal(D).astype(np.float32)
    h = tg.DeviceArray(D * 4)
    h.upload(h0)
    parr = (ctypes.c_void_p * layers)(*plans)
    step = lib.tg_hip_decode_create(ctypes.addressof(parr), layers, None, ctypes.c_float(1e-6), h.ptr,
                                    0 if args.no_graph else 1)
    if not step:
        raise RuntimeError(tg.last_error())

    for _ in range(args.warmup):
        lib.tg_hip_decode_run(step, None)
    lib.tg_hip_synchronize()
    t0 = time.perf_counter()
    ms = lib.tg_hip_decode_time(step, args.steps)
    lib.tg_hip_synchronize()
    wall = time.perf_counter() - t0
    ms_step = ms / args.steps
    bytes_step = layers * TOPK * EXPERT_B
    tok_s = 1e3 / ms_step
    log(f"timed {args.steps} steps: {ms:.2f} ms events, {wall * 1e3:.2f} ms wall")

    # per-kernel durations of one eager step (HIP events on the library stream)
    kms = (ctypes.c_float * 6)()
    kn = (ctypes.c_int * 6)()
    lib.tg_hip_decode_kernel_times(step, kms, kn)
    names = ["rms_norm", "quantize_x", "gate_up", "quantize_h", "down", "combine"]
    per_kernel = {names[i]: {"avg_us": round(kms[i] / max(kn[i], 1) * 1e3, 2), "launches": kn[i]}
                  for i in range(6)}
    gu_us = kms[2] / max(kn[2], 1) * 1e3
    gu_bytes = TOPK * 2 * GATE_B
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    traffic = read_traffic()
    log(f"kernels: {json.dumps(per_kernel)}")

    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "qwen3-30b-a3b expert decode step: 48 layers x top-8 of 128 resident experts, "
                        "D=2048 I=768, q4_K gate/up + q6_K down, batch 1, h += MoE(RMSNorm(h))",
            "layers": layers, "experts_per_layer": E, "top_k": TOPK, "embed_dim": D, "inter_dim": I,
            "resident_bytes": layers * E * EXPERT_B, "weight_bytes_per_step": bytes_step,
            "graph": not args.no_graph,
        },
        "weight_gbps": round(bytes_step / (ms_step * 1e-3) / 1e9, 1),
        "hbm_frac": round(bytes_step / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {
            "kernel": "k_moe_a<FQ4K,32> (gate+up+SiLU, 8 experts)",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "bytes_per_launch": gu_bytes, "avg_us": round(gu_us, 2),
        },
        "kernels": per_kernel,
        "device": name.value.decode(),
    }
    lib.tg_hip_decode_destroy(step)
    for p in plans:
        lib.tg_hip_moe_plan_destroy(p)
    for b in bufs:
        b.free()
    if not args.no_cpu:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(routes, min(args.cpu_layers, layers))
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
