#!/usr/bin/env python3
"""Training-step throughput of the byte Transformer on one MI355X.

Workload: BASELINE configs[1] (cfg2) -- 6-layer byte Transformer, d=384,
6 query / 2 KV heads (GQA), head_dim 64, SwiGLU 1024, causal, bf16 storage
with fp32 accumulation, batch 8 x seq 512 uniform random bytes, weights
N(0, 0.02), one full step = forward + backward + FP64 grad norm/clip +
AdamW (lr 3e-4, wd 0.01).  Inputs are resident in HBM before timing; the
step is replayed as a hipGraph (--no-graph for eager launches).

Prints ONE JSON line on stdout (the driver contract); progress goes to
stderr.  The roofline object covers the op with the largest share of the
step, timed live with HIP events on the model stream (one profiled eager
step after the timed region); the cpu_baseline object times the FP64 oracle
(a C restatement of the reference formulas, OpenMP) on a bounded sample.
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

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E


# single-kernel ops and the kernel each one launches (rocprofv3 names)
OP_KERNEL = {"attention_bwd_dkv": "k_attn_dkv_h", "attention_bwd_kv_reduce": "k_attn_kv_reduce", "attention_bwd_dq": "k_attn_dq", "attention_fwd": "k_attn_fwd",
             "adamw": "k_adamw_multi", "mirror_transpose": "k_transpose_jobs", "embedding_bwd": "k_embedding_bwd",
             "cross_entropy": "k_cross_entropy"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def op_work(op: str, mc, tc):
    """Algorithmic work of ONE launch of a step op: ("flop", F) or ("byte", B)."""
    M = tc.batch * tc.sequence
    d, F, V = mc.width, mc.ffn_width, 257
    J = mc.head_dim * mc.kv
    es = 2 if mc.precision == "bf16" else 4
    planes = mc.precision == "bf16" and mc.head_dim == 64 and os.environ.get("SJ_PLANES", "1") != "0"
    attn_fwd = tc.batch * mc.heads * 4 * mc.head_dim * tc.sequence * (tc.sequence + 1) / 2
    P = sum(math.prod(s) for _, s, _ in __import__("sejong_amd.model", fromlist=["layout"]).layout(mc))
    table = {
        "qkv_rope": ("flop", 2 * M * d * (d + 2 * J)),
        "qkv_dx": ("flop", 2 * M * d * (d + 2 * J)),
        "qkv_dw": ("flop", 2 * M * d * (d + 2 * J)),
        "attention_fwd": ("flop", attn_fwd),
        "attention_bwd": ("flop", 2.5 * attn_fwd),
        # split kernels: dQ recomputes S and dP and forms dQ (3 products of
        # the forward's size / 2); dK/dV recomputes S and dP, forms dV, dK (4)
        "attention_bwd_dq": ("flop", 1.5 * attn_fwd),
        "attention_bwd_dkv": ("flop", 2.0 * attn_fwd),
        # group sum of the per-head fp32 dK|dV partials, planes out
        "attention_bwd_kv_reduce": ("byte", (mc.heads // mc.kv) * M * 2 * J * 4 + 4 * M * 2 * J * 2),
        "mirror_transpose": ("byte", 2 * 2 * mc.layers * (d * (d + 2 * J) + d * d + 3 * d * F)),
        "attn_out_residual": ("flop", 2 * M * d * d),
        "attn_out_dx": ("flop", 2 * M * d * d),
        "attn_out_dw": ("flop", 2 * M * d * d),
        "gate_up_swiglu": ("flop", 2 * M * d * 2 * F),
        "gate_up_dx": ("flop", 2 * M * d * 2 * F),
        "gate_up_dw": ("flop", 2 * M * d * 2 * F),
        "down_residual": ("flop", 2 * M * F * d),
        "down_dx_swiglu": ("flop", 2 * M * F * d),
        "down_dw": ("flop", 2 * M * F * d),
        "head_fwd": ("flop", 2 * M * d * V),
        "head_dx": ("flop", 2 * M * d * V),
        "head_dw": ("flop", 2 * M * d * V),
        # plane path: y and y^T written; backward also writes hi/lo planes
        # in both orientations (4 bf16 copies of dx)
        "rmsnorm": ("byte", (3 if planes else 2) * M * d * es + d * es),
        "rmsnorm_bwd": ("byte", M * d * (es + 4 + 4 + 4 + (8 if planes else 0)) + d * es),
        "cross_entropy": ("byte", 2 * M * V * 4 + M * 8),
        "loss_summary": ("byte", M * 4),
        "embedding": ("byte", M * 4 + 2 * M * d * es),
        "embedding_bwd": ("byte", M * d * 4 + V * d * 4 + M * 4),
        "grad_norm": ("byte", P * 4),
        "adamw": ("byte", 30 * P),
    }
    return table.get(op, ("flop", 0.0))


def cpu_baseline(mc, tc, sample_batch: int):
    """FP64 oracle (OpenMP over all host threads) on `sample_batch`
    sequences of the same workload: forward + backward + AdamW."""
    import numpy as np
    from oracle import oracle as O
    from sejong_amd.model import byte_batch, init_params
    from sejong_amd.rng import Rng
    O.lib()
    p = init_params(mc, std=0.02).astype(np.float64)
    ids, tg = byte_batch(Rng(tc.seed), sample_batch, tc.sequence)
    cfg = dict(d=mc.width, layers=mc.layers, hq=mc.heads, hk=mc.kv, ffn=mc.ffn_width, T=tc.sequence,
               B=sample_batch, eps=mc.norm_epsilon, theta=mc.rope_theta)
    t0 = time.perf_counter()
    loss, g, _, _ = O.model_fwd_bwd(cfg, p, ids, tg, dtype=mc.precision)
    norm = math.sqrt(O.sum_squares(g))
    scale = min(1.0, tc.clip_norm / norm)
    O.adamw(p, g, np.zeros_like(p), np.zeros_like(p), tc.learning_rate, tc.beta1, tc.beta2, tc.epsilon,
            tc.weight_decay, 1 / (1 - tc.beta1), 1 / (1 - tc.beta2), scale)
    dt = time.perf_counter() - t0
    tokens = sample_batch * tc.sequence
    return {"value": tokens / dt, "unit": "tokens/s", "cores": O.num_threads(), "kind": "port",
            "sample": f"{sample_batch} of {tc.batch} sequences x {tc.sequence} bytes of the same workload "
                      f"(FP64 oracle fwd+bwd+AdamW, {dt:.2f} s)", "ms_per_step_sample": dt * 1e3}


def copy_probe(mib: int):
    """A plain copy of known size (reads and writes mib MiB) for scaling the
    FETCH_SIZE / WRITE_SIZE counters: one k_cast dispatch per repeat."""
    import ctypes
    from sejong_amd import _native as N
    N.load()
    n = mib * (1 << 20) // 4
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    N.api.sj_alloc(n * 4, ctypes.byref(a)); N.api.sj_alloc(n * 4, ctypes.byref(b))
    N.api.sj_fill(None, a, 0, n, ctypes.c_float(1.0))
    N.api.sj_synchronize(None)
    for _ in range(3):
        N.api.sj_cast(None, a, 0, b, 0, n)
    N.api.sj_synchronize(None)
    N.api.sj_free(a); N.api.sj_free(b)
    print(json.dumps({"copy_probe_bytes_read": n * 4, "copy_probe_bytes_written": n * 4, "dispatches": 3}),
          flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--cpu-sample-batch", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernels-json", default="", help="also write the per-op profile to this file")
    ap.add_argument("--profile-steps", type=int, default=5, help="eager steps timed op by op after the timed region")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain fp32 copy kernel (sj_cast) over this many MiB, 3 times, and exit: "
                         "the calibration for rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(each box has one GPU; sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.copy_probe_mib:
        copy_probe(args.copy_probe_mib)
        return

    import numpy as np
    from sejong_amd.model import Model, byte_batch, config, init_params
    from sejong_amd.rng import Rng

    mc, tc = config(args.config)
    tokens = tc.batch * tc.sequence
    log(f"[bench] {args.config}: d={mc.width} L={mc.layers} heads={mc.heads}/{mc.kv} ffn={mc.ffn_width} "
        f"B={tc.batch} T={tc.sequence} {mc.precision}, graph={not args.no_graph}")
    model = Model(mc, tc)
    model.set_params(init_params(mc, std=0.02, seed=mc.seed))
    ids, tg = byte_batch(Rng(tc.seed), tc.batch, tc.sequence)
    model.set_batch(ids, tg)  # resident in HBM before timing
    model.use_graph(not args.no_graph)

    for _ in range(args.warmup):
        model.train_step(tc.learning_rate)
    loss0, _ = model.read_loss()  # synchronises the model stream
    model.synchronize()
    t0 = time.perf_counter()
    gpu_ms = model.time_steps(args.steps, tc.learning_rate)  # HIP events around the K steps
    model.synchronize()
    wall = time.perf_counter() - t0
    loss, gnorm = model.read_loss()
    ms_per_step = max(gpu_ms, wall * 1e3) / args.steps
    log(f"[bench] {args.steps} steps: {ms_per_step:.4f} ms/step (events {gpu_ms / args.steps:.4f}, "
        f"wall {wall * 1e3 / args.steps:.4f}); loss {loss0:.5f} -> {loss:.5f}, |g| {gnorm:.4f}")

    # live per-op timing: eager steps with a HIP event pair around every op
    # on the model stream, averaged over the profiled steps
    model.profile(True)
    for _ in range(max(1, args.profile_steps)):
        model.train_step(tc.learning_rate)
    prof = model.profile_collect()
    model.profile(False)
    nprof = max(1, args.profile_steps)
    prof = {op: (ms / nprof, calls // nprof) for op, (ms, calls) in prof.items()}
    prof_total = sum(ms for ms, _ in prof.values())
    rows = []
    for op, (ms, calls) in sorted(prof.items(), key=lambda kv: -kv[1][0]):
        kind, work = op_work(op, mc, tc)
        avg_us = ms * 1e3 / calls
        rate = work / (avg_us * 1e-6) / 1e12 if kind == "flop" else work / (avg_us * 1e-6) / 1e9
        peak = PEAK_BF16_TFLOPS if kind == "flop" else PEAK_HBM_GBS
        rows.append({"op": op, "calls": calls, "avg_us": round(avg_us, 3), "share": round(ms / prof_total, 4),
                     "bound": "mfma" if kind == "flop" else "hbm",
                     "achieved": round(rate, 2), "unit": "TFLOP/s" if kind == "flop" else "GB/s",
                     "frac": round(rate / peak, 4)})
        log(f"  {op:20s} x{calls:3d} {avg_us:9.2f} us  {100 * ms / prof_total:5.1f}%  "
            f"{rate:9.2f} {'TFLOP/s' if kind == 'flop' else 'GB/s'}  ({100 * rate / peak:.1f}% of peak)")
    dom = rows[0]
    kind, work = op_work(dom["op"], mc, tc)
    # HBM bytes per dispatch of the dominant kernel, from the committed
    # rocprofv3 FETCH_SIZE / WRITE_SIZE runs (copy-kernel calibrated)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    kname = OP_KERNEL.get(dom["op"])
    if kname and os.path.exists(tpath):
        traffic = json.load(open(tpath)).get(args.config, {}).get("bytes_per_dispatch", {}).get(kname)
    roofline = {"bound": dom["bound"], "achieved": dom["achieved"],
                "peak": PEAK_BF16_TFLOPS if kind == "flop" else PEAK_HBM_GBS, "unit": dom["unit"],
                "frac": dom["frac"], "traffic": traffic, "op": dom["op"], "kernel": kname or dom["op"],
                "work_per_launch": work, "avg_launch_us": dom["avg_us"]}
    # whole-step MFMA fraction (algorithmic GEMM + attention flops / step time)
    step_flops = sum(op_work(op, mc, tc)[1] * calls for op, (_, calls) in prof.items()
                     if op_work(op, mc, tc)[0] == "flop")
    step_tflops = step_flops / (ms_per_step * 1e-3) / 1e12

    if args.kernels_json:
        with open(args.kernels_json, "w") as f:
            json.dump({"config": args.config, "ms_per_step": ms_per_step, "profile_step_ms": prof_total,
                       "ops": rows}, f, indent=1)

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (FP64 oracle) ...")
        cpu = cpu_baseline(mc, tc, args.cpu_sample_batch)
        log(f"[bench] cpu baseline {cpu['value']:.1f} tokens/s on {cpu['cores']} threads")

    out = {
        "metric": "train tokens/sec/GPU (fwd+bwd+update)",
        "value": round(tokens / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": mc.precision,
        "data": "synthetic uniform random bytes (SplitMix64 seed 123), weights N(0,0.02) seed 42",
        "config": {"workload": f"{args.config}: {mc.layers}-layer byte Transformer d{mc.width} GQA "
                               f"{mc.heads}/{mc.kv} hd{mc.head_dim} SwiGLU {mc.ffn_width}, fwd+bwd+AdamW",
                   "global_batch": tc.batch, "seq_len": tc.sequence, "tokens_per_step": tokens,
                   "parallelism": "single-gpu", "graph": not args.no_graph},
        "step_mfma": {"algorithmic_tflop_per_step": round(step_flops / 1e12, 4),
                      "achieved_tflops": round(step_tflops, 2), "frac": round(step_tflops / PEAK_BF16_TFLOPS, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "loss": loss,
    }
    print(json.dumps(out), flush=True)
    model.close()


if __name__ == "__main__":
    main()
