#!/usr/bin/env python3
"""Training-step throughput of the byte Transformer on one MI355X.

Workload: BASELINE configs[1] (cfg2) -- 6-layer byte Transformer, d=384,
6 query / 2 KV heads (GQA), head_dim 64, SwiGLU 1024, causal, bf16 storage
with fp32 accumulation, batch 8 x seq 512 uniform random bytes, weights
N(0, 0.02), one full step = forward + backward + FP64 grad norm/clip +
AdamW (lr 3e-4, wd 0.01).  Inputs are resident in HBM before timing; the
step is replayed as a hipGraph (--no-graph for eager launches).

Prints ONE JSON line on stdout (the driver contract); progress goes to
stderr.  The roofline object covers the kernel with the largest share of the
step's kernel time, timed live with HIP events on the model stream (eager
steps after the timed region); the cpu_baseline object times the FP64 oracle
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
# FP64 squared-norm slots the step's gradient producers wrote (0: the update
# read the whole gradient arena); set from the model after the timed steps
GRAD_SQ_SLOTS = 0


# op -> the one kernel it launches (rocprofv3 names) where the library does
# not name it itself (GEMM ops do, through the profile): the cfg2 step's
# plane-path kernels (bf16, head_dim 64, T a multiple of 64)
OP_KERNEL = {"attention_bwd": "k_attn2_bwd", "attention_bwd_dq_dkv": "k_attn2_bwd_g<3>", "attention_bwd_delta": "k_attn_delta",
             "attention_bwd_kv_reduce": "k_attn_kv_reduce_rows", "attention_fwd": "k_attn2_fwd<3>",
             "adamw": "k_adamw_tiles", "mirror_transpose": "k_transpose_jobs", "embedding_bwd": "k_embedding_bwd4",
             "embedding": "k_embedding_fwd", "cross_entropy": "k_cross_entropy_planes", "rmsnorm": "k_rms_fwd_t<3>",
             "rmsnorm_bwd": "k_rms_bwd_p<3>", "rmsnorm_dw_reduce": "k_rms_reduce_multi", "loss_summary": "k_loss_summary"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _attn_pairs(T, window):
    """(query, key) pairs a causal head visits: T(T+1)/2, or with a local
    window W < T, W(W+1)/2 + (T-W)W."""
    if window and window < T:
        return window * (window + 1) / 2 + (T - window) * window
    return T * (T + 1) / 2


def _hier_ops(mc, tc):
    """Per-step (kind, total work, calls) of every op of the hierarchical
    step (cfg3): the block ops summed over the three stages, the glue."""
    h = mc.hierarchy
    B, T, P = tc.batch, tc.sequence, h.patch_size
    Tg = -(-T // P)
    es = 2 if mc.precision == "bf16" else 4
    planes = mc.precision == "bf16"
    stages = [(h.encoder_layers, h.encoder_width, h.encoder_heads, h.encoder_heads, h.encoder_ffn_width, T,
               h.local_window),
              (mc.layers, mc.width, mc.heads, mc.kv, mc.ffn_width, Tg, 0),
              (h.decoder_layers, h.decoder_width, h.decoder_heads, h.decoder_heads, h.decoder_ffn_width, T,
               h.local_window)]
    # the library's row-layout dW rule: every stage on the transposed-operand
    # attention (T a multiple of 64) and no parameter-VJP groups
    rowdw = (planes and os.environ.get("SJ_ATTN_TT", "1") != "0" and all(s[5] % 64 == 0 for s in stages)
             and getattr(tc, "parameter_vjp", None) is None)
    tot = {}

    def add(op, kind, w, n=1):
        k, t, c = tot.get(op, (kind, 0.0, 0))
        tot[op] = (kind, t + w * n, c + n)
    for L, d, hq, hk, F, Ts, W in stages:
        M, J = B * Ts, d // hq * hk
        af = B * hq * 4 * (d // hq) * _attn_pairs(Ts, W)
        for op, kind, w in (("qkv_rope", "flop", 2 * M * d * (d + 2 * J)), ("qkv_dx", "flop", 2 * M * d * (d + 2 * J)),
                            ("qkv_dw", "flop", 2 * M * d * (d + 2 * J)), ("attention_fwd", "flop", af),
                            ("attention_bwd", "flop", 2.5 * af), ("attention_bwd_dq", "flop", 1.5 * af),
                            ("attention_bwd_dkv", "flop", 2.0 * af), ("attention_bwd_dq_dkv", "flop", 2.5 * af),
                            ("attention_bwd_delta", "byte", 3 * M * d * es + M * hq * 4),
                            ("attention_bwd_kv_reduce", "byte", (hq // hk) * M * 2 * J * 4 + 4 * M * 2 * J * 2),
                            ("attn_out_residual", "flop", 2 * M * d * d), ("attn_out_dx", "flop", 2 * M * d * d),
                            ("attn_out_dw", "flop", 2 * M * d * d), ("gate_up_swiglu", "flop", 4 * M * d * F),
                            ("gate_up_dx", "flop", 4 * M * d * F), ("gate_up_dw", "flop", 4 * M * d * F),
                            ("down_residual", "flop", 2 * M * F * d), ("down_dx_swiglu", "flop", 2 * M * F * d),
                            ("down_dw", "flop", 2 * M * F * d)):
            add(op, kind, w, L)
        tr = 0 if rowdw else 1  # transposed copies (y^T, dx planes^T) unless row-layout dW
        add("rmsnorm", "byte", (2 + (tr if planes else 0)) * M * d * es + d * es, 2 * L)
        add("rmsnorm", "byte", 2 * M * d * es + d * es)                       # closing norm
        add("rmsnorm_bwd", "byte", M * d * (es + 4 + 4 + 4 + (4 + 4 * tr if planes else 0)) + d * es, 2 * L)
        add("rmsnorm_bwd", "byte", M * d * (es + 4 + 4 + 4 + (4 + 4 * tr if planes else 0)) + d * es)
    de, dg, dd = h.encoder_width, mc.width, h.decoder_width
    Ml, Mg, V = B * T, B * Tg, 257
    for op, kind, w in (("patch_pool", "byte", Ml * de * es + Mg * de * es),
                        ("encoder_to_global", "flop", 2 * Mg * de * dg), ("global_to_decoder", "flop", 2 * Mg * dg * dd),
                        ("bos_to_decoder", "flop", 2 * dg * dd), ("patch_broadcast", "byte", Ml * dd * es + Mg * dd * es),
                        ("encoder_to_decoder", "flop", 2 * Ml * de * dd), ("decoder_input", "byte", 3 * Ml * dd * es),
                        ("output_projection", "flop", 2 * Ml * dd * dg), ("output_projection_dx", "flop", 2 * Ml * dd * dg),
                        ("output_projection_dw", "flop", 2 * Ml * dd * dg),
                        ("encoder_to_decoder_dx", "flop", 2 * Ml * de * dd), ("encoder_to_decoder_dw", "flop", 2 * Ml * de * dd),
                        ("patch_broadcast_bwd", "byte", Ml * dd * 4 + Mg * dd * 4 + dd * 4),
                        ("global_to_decoder_dw", "flop", 2 * Mg * dg * dd), ("bos_to_decoder_dw", "flop", 2 * dg * dd),
                        ("bos_to_decoder_dx", "flop", 2 * dg * dd), ("global_to_decoder_dx", "flop", 2 * Mg * dg * dd),
                        ("encoder_to_global_dx", "flop", 2 * Mg * de * dg), ("encoder_to_global_dw", "flop", 2 * Mg * de * dg),
                        ("patch_pool_bwd", "byte", Mg * de * 4 + Ml * de * 4), ("encoded_grad_sum", "byte", 3 * Ml * de * 4),
                        ("head_fwd", "flop", 2 * Ml * dg * V), ("head_dx", "flop", 2 * Ml * dg * V),
                        ("head_dw", "flop", 2 * Ml * dg * V), ("cross_entropy", "byte", 2 * Ml * V * 4 + Ml * 8),
                        ("loss_summary", "byte", Ml * 4), ("embedding", "byte", Ml * 4 + 2 * Ml * de * es),
                        ("embedding_bwd", "byte", Ml * de * 4 + V * de * 4 + Ml * 4)):
        add(op, kind, w)
    add("rmsnorm", "byte", 2 * Ml * dg * es + dg * es)                            # final norm
    add("rmsnorm_bwd", "byte", Ml * dg * (es + 4 + 4 + 4 + (4 if planes else 0)) + dg * es)
    if planes:  # the glue products' dY as hi/lo planes: one split pass each (fp32 in, two bf16 planes out)
        for n in (Ml * dd, Mg * dd, Mg * dg):
            add("glue_split", "byte", 8 * n)
    import sejong_amd.model as SM
    Pn = sum(math.prod(sh) for _, sh, _ in SM.layout(mc))
    mt = sum(L * (d * (d + 2 * (d // hq * hk)) + d * d + 3 * d * F) for L, d, hq, hk, F, _, _ in stages)
    add("grad_norm", "byte", Pn * 4)
    add("adamw", "byte", 30 * Pn)
    add("mirror_transpose", "byte", 2 * 2 * mt)
    return tot


def op_work(op: str, mc, tc):
    """Algorithmic work of ONE launch of a step op: ("flop", F) or ("byte", B)
    (for the hierarchical model: the op's per-step total over its launches
    divided by their number, the launches of one name differing by stage)."""
    if getattr(mc, "hierarchy", None) is not None:
        kind, total, calls = _hier_ops(mc, tc).get(op, ("flop", 0.0, 1))
        return kind, total / calls
    M = tc.batch * tc.sequence
    d, F, V = mc.width, mc.ffn_width, 257
    J = mc.head_dim * mc.kv
    es = 2 if mc.precision == "bf16" else 4
    planes = mc.precision == "bf16" and mc.head_dim == 64 and os.environ.get("SJ_PLANES", "1") != "0"
    # the library's row-layout dW rule (planes, transposed-operand attention,
    # no parameter-VJP groups): no transposed copies of the norm outputs
    rowdw = (planes and os.environ.get("SJ_ATTN_TT", "1") != "0" and tc.sequence % 64 == 0
             and getattr(tc, "parameter_vjp", None) is None)
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
        # one launch of both roles (the step's MFMA-layout attention): the
        # algorithmic backward is 2.5x the forward (dV, dP, dS->dQ, dK; the
        # S recompute of both roles is issued work, not counted)
        "attention_bwd_dq_dkv": ("flop", 2.5 * attn_fwd),
        "attention_bwd_delta": ("byte", 3 * M * d * es + M * mc.heads * 4),
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
        # plane path: y (and y^T unless the dW products read row layouts)
        # written; the backward also writes dx as hi/lo planes (and their
        # transposes unless row-layout dW)
        "rmsnorm": ("byte", (2 + (1 if planes and not rowdw else 0)) * M * d * es + d * es),
        # algorithmic (the dtypes used): x read, dy (fp32) read,
        # dx (fp32) written, plus the fused residual-gradient add's fp32 read;
        # the gradient planes it also writes are issued bytes (op_issued_bytes)
        "rmsnorm_bwd": ("byte", M * d * (es + 4 + 4 + 4) + d * es),
        "cross_entropy": ("byte", 2 * M * V * 4 + M * 8),
        "loss_summary": ("byte", M * 4),
        "embedding": ("byte", M * 4 + 2 * M * d * es),
        "embedding_bwd": ("byte", M * d * 4 + V * d * 4 + M * 4),
        # the arena, or the FP64 partials the gradient producers left
        "grad_norm": ("byte", 8 * GRAD_SQ_SLOTS if GRAD_SQ_SLOTS else P * 4),
        "adamw": ("byte", 30 * P),
    }

    ex = getattr(mc, "experts", None)
    if ex is not None:
        # MoE FFN (cfg4): S = M * top_k routed rows; the grouped expert
        # products count the routed rows only (not the 64-row segment padding)
        E, Fe, K = ex.count, ex.ffn_width, ex.top_k
        S = M * K
        cap = S + 63 * E
        table.update({
            "mirror_transpose": ("byte", 2 * 2 * mc.layers * (d * (d + 2 * J) + d * d + 3 * E * d * Fe)),
            "router_topk": ("flop", 2 * M * d * E), "router_dw": ("flop", 2 * M * d * E),
            "route_pack": ("byte", 2 * S * 4 * 2),
            "moe_gather": ("byte", 3 * S * d * 2),
            "expert_gate_up": ("flop", 2 * S * d * 2 * Fe), "expert_down": ("flop", 2 * S * Fe * d),
            "combine_residual": ("byte", S * d * 2 + 2 * M * d * 2),
            "combine_bwd": ("byte", S * d * 2 + M * d * 4 + 4 * cap * d * 2),
            "expert_down_dx_swiglu": ("flop", 2 * S * Fe * d), "expert_down_dw": ("flop", 2 * S * Fe * d),
            "expert_gate_up_dx": ("flop", 2 * S * d * 2 * Fe), "expert_gate_up_dw": ("flop", 2 * S * d * 2 * Fe),
            "gather_route_bwd": ("byte", S * d * 4 + 2 * M * d * 4),
        })
    pv = getattr(tc, "parameter_vjp", None)
    if pv is not None:
        # parameter VJP (cfg5): rank R, k selected rows; every layer has a
        # q|k|v and a gate|up group (the step driver checks the decisions)
        import ctypes

        from sejong_amd import _native as N
        out = [ctypes.c_long() for _ in range(3)]
        N.load()
        N.api.sj_pvjp_budget(pv.rank, pv.residual_fraction, pv.block_rows, M, d, F, *(ctypes.byref(o) for o in out))
        R, blocks, S = (o.value for o in out)
        k = S * pv.block_rows
        comp = mc.layers * (d * (d + 2 * J) + 2 * d * F)   # compressed parameters
        table.update({
            "pvjp_indices": ("byte", 4 * (F + blocks + R + k + d)),
            # R donor columns read (bf16) in each of the two passes, Q written twice
            "pvjp_basis": ("byte", 2 * (2 * M * R + 4 * M * R)),
            # X^T read for A = X^T Q and its k selected rows again, Q read,
            # E planes written
            "pvjp_prepare": ("byte", 2 * d * M + 2 * k * M + 8 * M * R + 4 * (R + k) * M),
            # E dY over the group's concatenated members (q|k|v and gate|up alternate)
            "pvjp_coefficients": ("flop", 2 * (R + k) * M * ((d + 2 * J) + 2 * F) / 2),
            # dense gradients read; factors are small
            "factored_norm": ("byte", 4 * (P - comp)),
            "norm_sum": ("byte", 0),
            # w read + written, bf16 mirror written, dense G read for the
            # uncompressed parameters
            "sgd_update": ("byte", 10 * P + 4 * (P - comp)),
        })
    elif getattr(tc, "optimizer", "adamw") == "sgd":
        table.update({"factored_norm": ("byte", 4 * P), "norm_sum": ("byte", 0), "sgd_update": ("byte", 14 * P)})
    return table.get(op, ("flop", 0.0))


def op_issued_bytes(op: str, mc, tc):
    """HBM bytes one launch of a bandwidth-bound op moves beyond its
    algorithmic bytes (op_work), or None: the RMSNorm backward's hi/lo
    gradient planes (and their transposes where the dW products read
    transposed copies); the AdamW update's transposed bf16 mirror of the
    projection matrices and the output head's hi/lo planes in both
    orientations (the bf16 planes models' update writes them itself)."""
    if getattr(mc, "hierarchy", None) is not None:
        return None
    M = tc.batch * tc.sequence
    d, F, V = mc.width, mc.ffn_width, 257
    J = mc.head_dim * mc.kv
    planes = mc.precision == "bf16" and mc.head_dim == 64 and os.environ.get("SJ_PLANES", "1") != "0"
    rowdw = (planes and os.environ.get("SJ_ATTN_TT", "1") != "0" and tc.sequence % 64 == 0
             and getattr(tc, "parameter_vjp", None) is None)
    if op == "rmsnorm_bwd" and planes:
        return M * d * (4 if rowdw else 8)
    if (op == "adamw" and planes and getattr(tc, "optimizer", "adamw") == "adamw"
            and os.environ.get("SJ_FUSED_ADAMW", "1") != "0"):
        ex = getattr(mc, "experts", None)
        ffn = 3 * d * (ex.count * ex.ffn_width if ex is not None else F)
        return 2 * mc.layers * (d * (d + 2 * J) + d * d + ffn) + 8 * d * ((V + 7) // 8 * 8)
    return None


# issued MFMA work of a kernel per unit of its algorithmic work: the GEMM
# kernels multiply hi/lo bf16 planes (PA x PB products, lo x lo skipped); the
# MFMA-layout attention kernels recompute S and dP and multiply the hi/lo
# planes of P, dO and dS (forward 3 products for the algorithmic 2; backward
# 13 for the algorithmic 5)
def issued_factor(kernel: str) -> float:
    if kernel.startswith("k_gemm_fast<"):
        t = [int(x) for x in kernel[len("k_gemm_fast<"):-1].split(",")]
        pa, pb = t[2], t[3]
        return float(pa * pb - (1 if pa == 2 and pb == 2 else 0))
    if kernel.startswith("k_gemm_kw<"):  # token-split dW: one X plane times PB planes of Y
        return float(int(kernel[len("k_gemm_kw<"):-1].split(",")[0]))
    return {"k_attn2_fwd<3>": 1.5, "k_attn2_bwd": 6.5 / 2.5, "k_attn2_bwd_g<3>": 6.5 / 2.5}.get(kernel, 1.0)


def kernel_roofline(prof, kern_only, op_kernel, mc, tc, config, kern_instep=None):
    """Roofline of the kernel with the largest share of the profiled step.

    Every op is charged to the kernel it launches: a GEMM op to the GEMM
    kernel the library names for it, with the time between the events that
    kernel recorded at its own start and end (no launch gaps, no split-K
    reduce); any other op to the one kernel of OP_KERNEL (else the op
    itself) with its event-bracketed time.  The dominant kernel's achieved
    rate is its algorithmic work summed over its launches divided by its
    summed time (the average work per launch over the average launch
    duration)."""
    per = {}
    for op, (ms, calls) in prof.items():
        kind, work = op_work(op, mc, tc)
        kern = op_kernel.get(op) or OP_KERNEL.get(op) or op
        kms = kern_only[op][0] if op in kern_only else ms
        e = per.setdefault(kern, {"ms": 0.0, "calls": 0, "work": 0.0, "kind": kind, "ops": []})
        e["ms"] += kms
        e["calls"] += calls
        e["work"] += work * calls
        e["ops"].append(op)
    total = sum(e["ms"] for e in per.values())
    top = sorted(per.items(), key=lambda kv: -kv[1]["ms"])[:8]
    log("  kernel time per launch: " + ", ".join(f"{k} {v['ms'] * 1e3 / v['calls']:.2f} us" for k, v in top))
    kern, e = max(per.items(), key=lambda kv: kv[1]["ms"])
    flop = e["kind"] == "flop"
    peak = PEAK_BF16_TFLOPS if flop else PEAK_HBM_GBS
    avg_us = e["ms"] * 1e3 / e["calls"]
    wpl = e["work"] / e["calls"]
    rate = wpl / (avg_us * 1e-6) / (1e12 if flop else 1e9)
    log(f"  dominant kernel {kern}: {100 * e['ms'] / total:.1f}% of the profiled kernel time, {e['calls']} launches "
        f"({', '.join(e['ops'])}), {avg_us:.2f} us, {rate:.2f} {'TFLOP/s' if flop else 'GB/s'}")
    # HBM bytes per dispatch of the dominant kernel, from the committed
    # rocprofv3 TCC EA-request runs
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get(config, {}).get("bytes_per_dispatch", {}).get(kern)
    out = {"bound": "mfma" if flop else "hbm", "achieved": round(rate, 2), "peak": peak,
           "unit": "TFLOP/s" if flop else "GB/s", "frac": round(rate / peak, 4), "traffic": traffic,
           "kernel": kern, "ops": e["ops"], "launches_per_step": e["calls"],
           "share_of_kernel_time": round(e["ms"] / total, 4), "work_per_launch": wpl, "avg_launch_us": round(avg_us, 3)}
    if flop:
        f = issued_factor(kern)
        out["issued"] = {"work_per_launch": wpl * f, "achieved": round(rate * f, 2), "frac": round(rate * f / peak, 4)}
    # the same kernel timed in the two-stream step (sharing the chip with the
    # other stream's kernels, as in the graph replay), beside the isolated time
    if kern_instep:
        ims = sum(kern_instep[op][0] for op in e["ops"] if op in kern_instep)
        icalls = sum(kern_instep[op][1] for op in e["ops"] if op in kern_instep)
        if icalls == e["calls"] and ims > 0:
            ius = ims * 1e3 / icalls
            irate = wpl / (ius * 1e-6) / (1e12 if flop else 1e9)
            out["in_step"] = {"avg_launch_us": round(ius, 3), "achieved": round(irate, 2),
                              "frac": round(irate / peak, 4)}
            log(f"  dominant kernel in the two-stream step: {ius:.2f} us per launch, {irate:.2f} "
                f"{'TFLOP/s' if flop else 'GB/s'}")
    return out


def _hier_name(name, mc):
    h = mc.hierarchy
    return (f"{name}: hierarchical byte model, encoder {h.encoder_layers}x d{h.encoder_width} and decoder "
            f"{h.decoder_layers}x d{h.decoder_width} (window {h.local_window}), global {mc.layers}x d{mc.width} "
            f"GQA {mc.heads}/{mc.kv} SwiGLU {mc.ffn_width} over {h.patch_size}-byte patches, ")


def cpu_sample_batch(mc, tc) -> int:
    """Sequences of the CPU baseline sample, sized for about 6-24 s of FP64
    work on the GPU box's 16 host threads (measured: cfg2 0.93 s per
    sequence, cfg3 1.6 s, cfg4 0.8 s, cfg5 24 s): the whole batch for cfg2
    and cfg4, 6 sequences of cfg3, 1 at width >= 1024 (cfg5)."""
    if mc.hierarchy is not None:
        return 6
    if mc.width >= 1024:
        return 1
    return tc.batch


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
    if getattr(mc, "experts", None) is not None:
        from oracle import moe as OM
        ex = mc.experts
        mcfg = dict(cfg, E=ex.count, K=ex.top_k, fe=ex.ffn_width)
        acts = OM.model_forward(mcfg, p, ids, mc.precision)
        loss, g, _ = OM.model_backward(mcfg, p, acts, ids, tg, mc.precision)
    elif mc.hierarchy is not None:
        from oracle import hierarchy as H
        h = mc.hierarchy
        hc = dict(cfg, P=h.patch_size, window=h.local_window, de=h.encoder_width, le=h.encoder_layers,
                  he=h.encoder_heads, fe=h.encoder_ffn_width, dd=h.decoder_width, ld=h.decoder_layers,
                  hd=h.decoder_heads, fd=h.decoder_ffn_width)
        acts = H.model_forward(hc, p, ids, mc.precision)
        loss, g = H.model_backward(hc, p, acts, ids, tg, mc.precision)
    else:
        loss, g, _, _ = O.model_fwd_bwd(cfg, p, ids, tg, dtype=mc.precision)
    norm = math.sqrt(O.sum_squares(g))
    scale = min(1.0, tc.clip_norm / norm)
    if getattr(tc, "optimizer", "adamw") == "sgd":
        # dense-gradient SGD update (the oracle has no factored step)
        p -= tc.learning_rate * scale * g
        what = "FP64 oracle fwd+bwd with dense gradients + SGD"
    else:
        O.adamw(p, g, np.zeros_like(p), np.zeros_like(p), tc.learning_rate, tc.beta1, tc.beta2, tc.epsilon,
                tc.weight_decay, 1 / (1 - tc.beta1), 1 / (1 - tc.beta2), scale)
        what = "FP64 oracle fwd+bwd+AdamW"
    dt = time.perf_counter() - t0
    tokens = sample_batch * tc.sequence
    out = {"value": tokens / dt, "unit": "tokens/s", "cores": O.num_threads(), "kind": "port",
           "sample": f"{sample_batch} of {tc.batch} sequences x {tc.sequence} bytes of the same workload "
                     f"({what}, {dt:.2f} s)", "ms_per_step_sample": dt * 1e3, "cpu_model": _cpu_model()}
    if mc.hierarchy is None and getattr(mc, "experts", None) is None and mc.width < 1024:
        out.update(cpu_extras(mc, tc))
    return out


def _cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with its family / model /
    stepping numbers (a virtualised host may report only a generic name) and
    the logical CPUs this process may run on."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("model name", "cpu family", "model", "stepping", "cpu MHz") and k not in info:
                info[k] = v.strip()
            if k == "processor" and info:
                break
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    try:
        ncpu = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        ncpu = os.cpu_count() or 0
    return (f"{name} (family {info.get('cpu family', '?')} model {info.get('model', '?')} stepping "
            f"{info.get('stepping', '?')}, {info.get('cpu MHz', '?')} MHz, {ncpu} logical CPUs available)")


def cpu_extras(mc, tc) -> dict:
    """The rest of the CPU plan: the cfg1 step (fp32 block, fwd+bwd+AdamW)
    and per-kernel FP64 oracle times at this workload's shapes (RMSNorm
    forward/backward, grouped attention forward/backward, AdamW over every
    parameter), all on the same host threads."""
    import numpy as np
    from oracle import oracle as O
    from sejong_amd.model import byte_batch, config, init_params, param_count
    from sejong_amd.rng import Rng

    def timed(f, reps=1):
        t = time.perf_counter()
        for _ in range(reps):
            f()
        return (time.perf_counter() - t) * 1e3 / reps

    m1, t1 = config("cfg1")
    p1 = init_params(m1, std=0.02).astype(np.float64)
    i1, g1 = byte_batch(Rng(t1.seed), t1.batch, t1.sequence)
    c1 = dict(d=m1.width, layers=m1.layers, hq=m1.heads, hk=m1.kv, ffn=m1.ffn_width, T=t1.sequence, B=t1.batch,
              eps=m1.norm_epsilon, theta=m1.rope_theta)

    def cfg1_step():
        loss, g, _, _ = O.model_fwd_bwd(c1, p1, i1, g1, dtype="f32")
        sc = min(1.0, t1.clip_norm / math.sqrt(O.sum_squares(g)))
        O.adamw(p1.copy(), g, np.zeros_like(p1), np.zeros_like(p1), t1.learning_rate, t1.beta1, t1.beta2,
                t1.epsilon, t1.weight_decay, 1 / (1 - t1.beta1), 1 / (1 - t1.beta2), sc)
    cfg1_ms = timed(cfg1_step, 3)
    rng = np.random.default_rng(0)
    M, d, Dh, B, T = tc.batch * tc.sequence, mc.width, mc.head_dim, tc.batch, tc.sequence
    x = rng.normal(0, 1, (M, d)); w = np.ones(d); dy = rng.normal(0, 1e-3, (M, d))
    q = rng.normal(0, 1, (M, mc.heads * Dh)); k = rng.normal(0, 1, (M, mc.kv * Dh)); v = rng.normal(0, 1, (M, mc.kv * Dh))
    o, lse = O.attention_fwd(q, k, v, B, T, mc.heads, mc.kv, Dh)
    do = rng.normal(0, 1e-3, o.shape)
    n = param_count(mc)
    pw, ppw = O._d(rng.normal(0, 0.02, n)); pg, ppg = O._d(rng.normal(0, 1e-3, n))
    pm, ppm = O._d(np.zeros(n)); pv, ppv = O._d(np.zeros(n))
    kern = {
        "rmsnorm_fwd": timed(lambda: O.rmsnorm_fwd(x, w, mc.norm_epsilon), 3),
        "rmsnorm_bwd": timed(lambda: O.rmsnorm_bwd(x, w, dy, mc.norm_epsilon), 3),
        "attention_fwd": timed(lambda: O.attention_fwd(q, k, v, B, T, mc.heads, mc.kv, Dh)),
        "attention_bwd": timed(lambda: O.attention_bwd(q, k, v, o, lse, do, B, T, mc.heads, mc.kv, Dh)),
        "adamw": timed(lambda: O.lib().or_adamw(ppw, ppg, ppm, ppv, n, tc.learning_rate, tc.beta1, tc.beta2,
                                                tc.epsilon, tc.weight_decay, 1 / (1 - tc.beta1),
                                                1 / (1 - tc.beta2), 1.0), 3),
    }
    return {"cfg1_step_ms": round(cfg1_ms, 3),
            "cfg1_tokens_per_s": round(t1.batch * t1.sequence / (cfg1_ms * 1e-3), 1),
            "kernel_ms": {kk: round(vv, 3) for kk, vv in kern.items()},
            "kernel_shapes": f"rmsnorm [{M}x{d}]; attention B{B} T{T} heads {mc.heads}/{mc.kv} hd{Dh}; "
                             f"adamw over {n} parameters"}


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


def copy_reference(byte_counts, reps: int = 9):
    """The practical ceiling of a bandwidth-bound op of a given size: the
    library's plain copy (k_cast, fp32 -> fp32) moving the same bytes, half
    read and half written, timed hot and with the cold-cache pass's 512 MiB
    write in front of it.  That write leaves dirty lines in the 256 MB
    Infinity Cache whose write-back the next kernel pays for, so a cold copy
    runs well below a hot one.  Returns {bytes: (hot_us, cold_us)}, medians."""
    import ctypes
    import statistics
    from sejong_amd import _native as N
    api = N.api
    keep = []
    top = max(byte_counts)
    half = (top // 2 + 15) // 16 * 16
    src, dst = _Buf(api, half, keep), _Buf(api, half, keep)
    flush_n = 512 * (1 << 20) // 4
    flush = _Buf(api, flush_n * 4, keep)
    api.sj_fill(None, src.p(), 0, half // 4, ctypes.c_float(1.0))
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    api.sj_event_create(ctypes.byref(a)); api.sj_event_create(ctypes.byref(b))
    ms = ctypes.c_float()
    out = {}
    try:
        for nbytes in byte_counts:
            n = max(nbytes // 8, 1)  # fp32 elements read (and written)
            times = {False: [], True: []}
            for cold in (False, True):
                for i in range(reps + 2):
                    if cold:
                        api.sj_fill(None, flush.p(), 0, flush_n, ctypes.c_float(0.0))
                    api.sj_event_record(a, None)
                    api.sj_cast(None, src.p(), 0, dst.p(), 0, n)
                    api.sj_event_record(b, None)
                    api.sj_event_elapsed(a, b, ctypes.byref(ms))
                    if i >= 2:
                        times[cold].append(ms.value * 1e3)
            out[nbytes] = (statistics.median(times[False]), statistics.median(times[True]))
    finally:
        api.sj_event_destroy(a); api.sj_event_destroy(b)
        for buf in keep:
            api.sj_free(buf.p())
    return out


# ------------------------------------------------------------ workloads
class _Buf:
    """A device buffer from the library allocator (torch is not loaded:
    its wheel carries a second HIP runtime)."""

    def __init__(self, api, nbytes, keep):
        import ctypes
        self.api = api
        p = ctypes.c_void_p()
        api.sj_alloc(max(int(nbytes), 256), ctypes.byref(p))
        self.ptr = p.value
        self.nbytes = int(nbytes)
        keep.append(self)

    def p(self, offset_bytes=0):
        import ctypes
        return ctypes.c_void_p(self.ptr + offset_bytes)

    def upload(self, arr):
        import ctypes
        import numpy as np
        a = np.ascontiguousarray(arr)
        self.api.sj_upload(self.p(), ctypes.c_void_p(a.ctypes.data), a.nbytes)
        return self


def _bf16(x):
    import numpy as np
    return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


class _OpTimer:
    """HIP events around each op on the NULL stream (one profiled pass)."""

    def __init__(self, api):
        self.api, self.events, self.names = api, [], []

    def op(self, name, fn):
        import ctypes
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        self.api.sj_event_create(ctypes.byref(a)); self.api.sj_event_create(ctypes.byref(b))
        self.api.sj_event_record(a, None)
        fn()
        self.api.sj_event_record(b, None)
        self.events.append((a, b)); self.names.append(name)

    def collect(self):
        import ctypes
        self.api.sj_synchronize(None)
        out = {}
        for name, (a, b) in zip(self.names, self.events):
            ms = ctypes.c_float()
            self.api.sj_event_elapsed(a, b, ctypes.byref(ms))
            t, c = out.get(name, (0.0, 0))
            out[name] = (t + ms.value, c + 1)
            self.api.sj_event_destroy(a); self.api.sj_event_destroy(b)
        return out


def _time_region(api, fn, steps):
    import ctypes
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    api.sj_event_create(ctypes.byref(a)); api.sj_event_create(ctypes.byref(b))
    api.sj_synchronize(None)
    t0 = time.perf_counter()
    api.sj_event_record(a, None)
    for _ in range(steps):
        fn(None)
    api.sj_event_record(b, None)
    api.sj_synchronize(None)
    wall = time.perf_counter() - t0
    ms = ctypes.c_float()
    api.sj_event_elapsed(a, b, ctypes.byref(ms))
    api.sj_event_destroy(a); api.sj_event_destroy(b)
    return max(ms.value, wall * 1e3) / steps


def _report(metric, unit, value, ms, args, config, prof, work, dtype, extra=None):
    rows = []
    total = sum(t for t, _ in prof.values())
    for op, (t, c) in sorted(prof.items(), key=lambda kv: -kv[1][0]):
        kind, w = work.get(op, ("flop", 0.0))
        avg_us = t * 1e3 / c
        rate = w / (avg_us * 1e-6) / (1e12 if kind == "flop" else 1e9)
        peak = PEAK_BF16_TFLOPS if kind == "flop" else PEAK_HBM_GBS
        rows.append(dict(op=op, calls=c, avg_us=avg_us, kind=kind, rate=rate, frac=rate / peak, work=w))
        log(f"  {op:24s} x{c:3d} {avg_us:9.2f} us  {100 * t / total:5.1f}%  {rate:9.2f} "
            f"{'TFLOP/s' if kind == 'flop' else 'GB/s'}  ({100 * rate / peak:.1f}% of peak)")
    dom = rows[0]
    out = {"metric": metric, "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": dtype, "data": "synthetic (numpy seeded normal / SplitMix64 draws)",
           "config": config,
           "roofline": {"bound": "mfma" if dom["kind"] == "flop" else "hbm", "achieved": round(dom["rate"], 2),
                        "peak": PEAK_BF16_TFLOPS if dom["kind"] == "flop" else PEAK_HBM_GBS,
                        "unit": "TFLOP/s" if dom["kind"] == "flop" else "GB/s", "frac": round(dom["frac"], 4),
                        "traffic": None, "op": dom["op"], "work_per_launch": dom["work"],
                        "avg_launch_us": round(dom["avg_us"], 3)},
           "cpu_baseline": None}
    if extra:
        out.update(extra)
    print(json.dumps(out), flush=True)


def workload_moe(args):
    """cfg4: the MoE FFN of 4 layers, d 512, 8 SwiGLU
    experts of width 1024, top-2, 4096 tokens: router + top-k, device pack,
    grouped gate/up and down, combine + residual; the backward (combine,
    grouped down dX + SwiGLU, grouped dW, grouped gate/up dX, gather +
    routing backward + router dW); AdamW on the fp32 expert masters and
    the bf16 mirror cast.  The forms the training step runs: the grouped dW
    on the row-layout operands (packed rows and the dX chain's planes), no
    transposed copies.  Attention is not part of this measurement."""
    import ctypes
    import numpy as np
    from sejong_amd import _native as N
    lib = N.load(); api = N.api
    L, M, d, E, F, K = 4, 4096, 512, 8, 1024, 2
    cf = ctypes.c_float
    keep = []
    rng = np.random.default_rng(0)
    B = lambda nbytes: _Buf(api, nbytes, keep)
    cap = lib.sj_route_pack_capacity(M * K, E)
    S = M * K
    layers = []
    for l in range(L):
        wg = rng.normal(0, 0.02, (E, d, F)); wu = rng.normal(0, 0.02, (E, d, F)); wd = rng.normal(0, 0.02, (E, F, d))
        gu = np.concatenate([wg, wu], 2).astype(np.float32)                    # [E][d][2F]
        master = np.concatenate([gu.ravel(), wd.astype(np.float32).ravel()])
        P = master.size
        y = dict(P=P)
        y["w"] = B(P * 4).upload(master); y["g"] = B(P * 4); y["m"] = B(P * 4).upload(np.zeros(P, np.float32))
        y["v"] = B(P * 4).upload(np.zeros(P, np.float32)); y["mirror"] = B(P * 2).upload(_bf16(master))
        y["gu_t"] = B(E * 2 * F * d * 2).upload(_bf16(np.concatenate([wg.transpose(0, 2, 1), wu.transpose(0, 2, 1)], 1)))
        y["d_t"] = B(E * d * F * 2).upload(_bf16(wd.transpose(0, 2, 1)))
        y["wr"] = B(d * E * 2).upload(_bf16(rng.normal(0, d ** -0.5, (d, E))))
        layers.append(y)
    z = B(M * d * 2).upload(_bf16(rng.normal(0, 1, (M, d)))); x1 = B(M * d * 2).upload(_bf16(rng.normal(0, 1, (M, d))))
    out = B(M * d * 2)
    logits, ids, wts = B(M * E * 2), B(S * 4), B(S * 4)
    tok, slt, cnt, off, ps, pp = B(E * S * 4), B(E * S * 4), B(E * 4), B((E + 1) * 4), B(cap * 4), B(S * 4)
    zp = B(cap * d * 2)
    g_, u_, h_ = B(cap * F * 2), B(cap * F * 2), B(cap * F * 2)
    yp = B(cap * d * 2)
    dres = B(M * d * 4).upload(rng.normal(0, 1e-3, (M, d)).astype(np.float32))
    dxh, dxl = (B(cap * d * 2) for _ in range(2))
    dwts = B(S * 4)
    dgh, dgl = (B(cap * 2 * F * 2) for _ in range(2))
    dzp, dz, dlog, dwr = B(cap * d * 4), B(M * d * 4), B(M * E * 4), B(d * E * 4)
    ws = B(max(lib.sj_gemm_workspace_bytes(d, E, M), 256))
    api.sj_synchronize(None)

    def step(T):
        run = (lambda n, f: T.op(n, f)) if T else (lambda n, f: f())
        for y in layers:
            run("router_topk", lambda: api.sj_router_topk(None, z.p(), d, y["wr"].p(), d, M, E, K, logits.p(), ids.p(), wts.p()))
            run("route_pack", lambda: api.sj_route_pack(None, ids.p(), M, K, E, tok.p(), slt.p(), cnt.p(), off.p(), ps.p(), pp.p(), cap))
            run("moe_gather", lambda: api.sj_moe_gather(None, z.p(), d, d, ps.p(), K, cap, zp.p(), None, cap))
            run("expert_gate_up", lambda: api.sj_moe_gate_up_fwd(None, off.p(), E, cap, zp.p(), d, d, y["gu_t"].p(), y["gu_t"].p(F * d * 2), d, 2 * F * d, F, g_.p(), u_.p(), h_.p(), F, None, cap))
            run("expert_down", lambda: api.sj_moe_down_fwd(None, off.p(), E, cap, h_.p(), F, F, y["d_t"].p(), F, d * F, d, yp.p(), d))
            run("combine_residual", lambda: api.sj_moe_combine(None, yp.p(), d, d, ids.p(), pp.p(), wts.p(), M, K, x1.p(), d, out.p(), d))
        for y in reversed(layers):
            gu_off = E * d * 2 * F
            run("combine_bwd", lambda: api.sj_moe_combine_bwd(None, yp.p(), d, d, ps.p(), wts.p(), K, cap, dres.p(), d, dxh.p(), dxl.p(), None, None, cap, dwts.p()))
            run("expert_down_dx_swiglu", lambda: api.sj_moe_down_bwd_swiglu_p(None, off.p(), E, cap, dxh.p(), dxl.p(), d, d, y["mirror"].p(gu_off * 2), d, F * d, F, g_.p(), u_.p(), F, dgh.p(), dgl.p(), 2 * F, None, None, cap))
            run("expert_down_dw", lambda: api.sj_moe_gemm_dw_tn(None, off.p(), E, cap, F, d, h_.p(), F, dxh.p(), dxl.p(), d, y["g"].p(gu_off * 4), d, F * d))
            run("expert_gate_up_dx", lambda: api.sj_moe_gemm_rows(None, off.p(), E, cap, d, 2 * F, dgh.p(), dgl.p(), 2 * F, y["mirror"].p(), 2 * F, d * 2 * F, dzp.p(), d, 0))
            run("expert_gate_up_dw", lambda: api.sj_moe_gemm_dw_tn(None, off.p(), E, cap, d, 2 * F, zp.p(), d, dgh.p(), dgl.p(), 2 * F, y["g"].p(), 2 * F, d * 2 * F))
            run("gather_route_bwd", lambda: api.sj_moe_gather_bwd(None, dzp.p(), d, d, ids.p(), pp.p(), wts.p(), logits.p(), dwts.p(), y["wr"].p(), M, K, E, dres.p(), d, dz.p(), d, dlog.p()))
            run("router_dw", lambda: api.sj_gemm(None, 1, 0, d, E, M, z.p(), 4, d, dlog.p(), 0, E, dwr.p(), 0, E, 0, ws.p(), ws.nbytes))
        for y in layers:
            run("expert_adamw", lambda: api.sj_adamw(None, y["w"].p(), y["g"].p(), y["m"].p(), y["v"].p(), y["P"], cf(3e-4), cf(0.9), cf(0.95), cf(0.0), cf(0.01), cf(10.0), cf(20.0), cf(1.0)))
            run("mirror_cast", lambda: api.sj_cast(None, y["w"].p(), 0, y["mirror"].p(), 4, y["P"]))

    for _ in range(args.warmup):
        step(None)
    ms = _time_region(api, step, args.steps)
    T = _OpTimer(api)
    step(T)
    prof = T.collect()
    Pexp = layers[0]["P"]
    work = {"expert_gate_up": ("flop", 2 * S * d * 2 * F), "expert_down": ("flop", 2 * S * F * d),
            "expert_down_dx_swiglu": ("flop", 2 * S * F * d), "expert_down_dw": ("flop", 2 * S * F * d),
            "expert_gate_up_dx": ("flop", 2 * S * d * 2 * F), "expert_gate_up_dw": ("flop", 2 * S * d * 2 * F),
            "router_topk": ("flop", 2 * M * d * E), "router_dw": ("flop", 2 * M * d * E),
            "expert_adamw": ("byte", 28 * Pexp), "mirror_cast": ("byte", 6 * Pexp),
            "moe_gather": ("byte", 3 * M * K * d * 2), "combine_residual": ("byte", M * K * d * 2 + 2 * M * d * 2),
            "combine_bwd": ("byte", M * K * d * 2 + M * d * 4 + 4 * cap * d * 2),
            "gather_route_bwd": ("byte", M * K * d * 4 + 2 * M * d * 4), "route_pack": ("byte", 2 * S * 4 * 2)}
    flops = L * 3 * (2 * S * d * 2 * F + 2 * S * F * d)
    log(f"[bench moe] {args.steps} steps: {ms:.4f} ms/step; grouped expert GEMM {flops / 1e9:.1f} GF/step "
        f"-> {flops / (ms * 1e-3) / 1e12:.1f} TFLOP/s")
    _report("MoE FFN train tokens/sec (grouped-GEMM fwd+bwd + expert AdamW)", "tokens/s", M / (ms * 1e-3), ms, args,
            {"workload": "cfg4 MoE FFN: 4 layers, d512, 8 SwiGLU experts x 1024, top-2, 4096 tokens, bf16 "
                         "(attention excluded)", "global_batch": 8, "seq_len": 512, "parallelism": "single-gpu"},
            prof, work, "bf16",
            {"expert_gemm_mfma": {"algorithmic_tflop_per_step": round(flops / 1e12, 4),
                                  "achieved_tflops": round(flops / (ms * 1e-3) / 1e12, 2)}})


def workload_pvjp(args):
    """cfg5 parameter-VJP pieces of one step: 16384
    tokens, d 1024, 12 layers, FFN 2752, rank 16, 10% of 32-row blocks.  One
    index draw and one basis (shared by all groups: same n, rank and width),
    a prepare per projection group (QKV and gate/up of 12 layers) on the
    stored input rows and a coefficient GEMM per group on the row-layout dY
    planes (the forms the training step runs),
    the coefficient GEMM of every compressed member (q, k, v, gate, up), and
    the factored SGD update over all 133.5M parameters (dense gradients for
    the single-use projections, embedding, norms and head).  The dense
    model's own forward/backward GEMMs are not part of this measurement."""
    import ctypes
    import numpy as np
    from sejong_amd import _native as N
    lib = N.load(); api = N.api
    n, d, F, L, HQ, HK, V = 16384, 1024, 2752, 12, 16, 4, 257
    J = d // HQ * HK
    cf = ctypes.c_float
    keep = []
    B = lambda nbytes: _Buf(api, nbytes, keep)
    rng = np.random.default_rng(1)
    R, blocks, S = 16, 32, 4
    k = S * 32
    seed = 0x1234
    # donor: the up projection's output u [n][F] (widest member of the gate/up
    # group, the last one on ties)
    donor = B(n * F * 2).upload(_bf16(rng.normal(0, 1, (n, F))))
    x = B(n * d * 2).upload(_bf16(rng.normal(0, 1, (n, d))))
    scr, cols, rows_, fmap = B((F + blocks) * 4), B(R * 4), B(k * 4), B(d * 4)
    q = B(n * R * 4)
    wsb = B(lib.sj_pvjp_basis_workspace_bytes(n, R))
    eps = lib.sj_pvjp_basis_tolerance(n, R)
    groups = []
    for g in range(2 * L):
        groups.append(dict(left=B(d * R * 4), e=B((R + k) * n * 4), eh=B((R + k) * n * 2), el=B((R + k) * n * 2)))
    # dY planes of a group's members, concatenated as the step keeps them
    # ([tokens][q|k|v] and [tokens][gate|up]): one coefficient GEMM per group
    W2 = 2 * F
    dyh = B(W2 * n * 2).upload(_bf16(rng.normal(0, 1e-4, (n, W2))))
    dyl = B(W2 * n * 2).upload(np.zeros(W2 * n, np.uint16))
    wsp = B(max(lib.sj_pvjp_prepare_workspace_bytes(d, n, R), lib.sj_pvjp_vjp_workspace_bytes(R + k, W2, n), 256))
    # parameters (reference layout shapes) and their gradients
    members = []   # (rows, cols, group index or None, member width)
    shapes = [("embedding", V, d, None)]
    for l in range(L):
        shapes += [("an", 1, d, None), ("fn", 1, d, None), ("q", d, d, 2 * l), ("k", d, J, 2 * l), ("v", d, J, 2 * l),
                   ("o", d, d, None), ("gate", d, F, 2 * l + 1), ("up", d, F, 2 * l + 1), ("down", F, d, None)]
    shapes += [("final_norm", 1, d, None), ("output", d, V, None)]
    total = sum(r * c for _, r, c, _ in shapes)
    params, terms, coeffs = [], [], []
    # coefficients per group [R+k][sum of member widths]; a member's right /
    # tail are column slices of it (row stride = the group width)
    gwidth = {}
    for name, r, c, gi in shapes:
        if gi is not None:
            gwidth[gi] = gwidth.get(gi, 0) + c
    gco = {gi: B((R + k) * wdt * 4) for gi, wdt in gwidth.items()}
    coeffs = [(gi, gco[gi], wdt) for gi, wdt in sorted(gwidth.items())]
    col0 = {}
    for name, r, c, gi in shapes:
        w = B(r * c * 4).upload(rng.normal(0, 0.02, r * c).astype(np.float32))
        if gi is None:
            dense = B(r * c * 4).upload(rng.normal(0, 1e-4, r * c).astype(np.float32))
            params.append(N.FactoredParam(w.ptr, dense.ptr, r, c, int(r > 1), 0, 0))
        else:
            off = col0.get(gi, 0); col0[gi] = off + c
            base, wdt = gco[gi].ptr, gwidth[gi]
            terms.append(N.FactoredTerm(groups[gi]["left"].ptr, base + off * 4, base + (R * wdt + off) * 4, fmap.ptr,
                                        R, 1.0, wdt))
            params.append(N.FactoredParam(w.ptr, None, r, c, 1, len(terms) - 1, 1))
    PA = (N.FactoredParam * len(params))(*params)
    TA = (N.FactoredTerm * len(terms))(*terms)
    nbytes = lib.sj_factored_meta_bytes(PA, len(params), len(terms))
    host = np.zeros(nbytes, np.uint8)
    tiles = ctypes.c_long()
    api.sj_factored_pack(PA, len(params), TA, len(terms), ctypes.c_void_p(host.ctypes.data), nbytes, ctypes.byref(tiles))
    meta = B(nbytes).upload(host)
    part, norm = B(tiles.value * 8), B(8)
    api.sj_synchronize(None)

    def step(T):
        run = (lambda nm, f: T.op(nm, f)) if T else (lambda nm, f: f())
        run("pvjp_indices", lambda: api.sj_pvjp_indices(None, seed, d, F, blocks, S, R, 32, scr.p(), cols.p(), rows_.p(), fmap.p()))
        run("pvjp_basis", lambda: api.sj_pvjp_basis(None, donor.p(), 4, F, n, cols.p(), R, cf(eps), q.p(), wsb.p(), wsb.nbytes))
        for g in groups:
            run("pvjp_prepare", lambda: api.sj_pvjp_prepare_rows(None, x.p(), d, d, n, q.p(), R, rows_.p(), k, cf(blocks / S), g["left"].p(), g["e"].p(), g["eh"].p(), g["el"].p(), n, wsp.p(), wsp.nbytes))
        for gi, co, c in coeffs:
            g = groups[gi]
            run("pvjp_coefficients", lambda: api.sj_pvjp_vjp_rows(None, g["eh"].p(), g["el"].p(), n, R + k, n, dyh.p(), dyl.p(), W2, c, co.p(), c, wsp.p(), wsp.nbytes))
        run("factored_norm", lambda: api.sj_factored_apply(None, meta.p(), tiles.value, 2, cf(0), cf(0), part.p()))
        run("norm_sum", lambda: api.sj_sum_f64(None, part.p(), tiles.value, norm.p()))
        run("factored_sgd_update", lambda: api.sj_factored_apply(None, meta.p(), tiles.value, 1, cf(1e-2), cf(0.0), None))

    for _ in range(args.warmup):
        step(None)
    ms = _time_region(api, step, args.steps)
    T = _OpTimer(api)
    step(T)
    prof = T.collect()
    dense_params = sum(r * c for _, r, c, gi in shapes if gi is None)
    upd_bytes = 8 * total + 4 * dense_params
    avg_b = sum(c for _, _, c in coeffs) / len(coeffs)
    work = {"pvjp_prepare": ("flop", 2 * d * R * n), "pvjp_coefficients": ("flop", 2 * (R + k) * avg_b * n),
            "factored_sgd_update": ("byte", upd_bytes), "factored_norm": ("byte", 4 * total + 4 * dense_params),
            "pvjp_basis": ("byte", n * R * 4 * 2), "pvjp_indices": ("byte", d * 4), "norm_sum": ("byte", tiles.value * 8)}
    log(f"[bench pvjp] {args.steps} steps: {ms:.4f} ms/step; {total / 1e6:.2f}M parameters, factored update "
        f"{upd_bytes / 1e9:.2f} GB")
    _report("parameter-VJP pieces per training step (tokens/s)", "tokens/s", n / (ms * 1e-3), ms, args,
            {"workload": "cfg5 parameter-VJP pieces: 16384 tokens, d1024, 12 layers, FFN 2752, rank 16, 10% of "
                         "32-row blocks (indices + basis + 24 prepares + 60 coefficient GEMMs + factored SGD over "
                         f"{total / 1e6:.2f}M params; dense forward/backward excluded)",
             "global_batch": 16, "seq_len": 1024, "parallelism": "single-gpu"},
            prof, work, "f32")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--cpu-sample-batch", type=int, default=0,
                    help="sequences the CPU baseline runs (default: cpu_sample_batch, about 10 s of FP64 work)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernels-json", default="", help="also write the per-op profile to this file")
    ap.add_argument("--profile-steps", type=int, default=5, help="eager steps timed op by op after the timed region (then as many with each GEMM kernel timed alone)")
    ap.add_argument("--cold-steps", type=int, default=1,
                    help="eager steps timed op by op with a 512 MiB cache flush before every op (0: skip)")
    ap.add_argument("--workload", default="step", choices=["step", "moe", "pvjp"],
                    help="step: the cfg2 training step (default, the headline); moe: the cfg4 MoE FFN; "
                         "pvjp: the cfg5 parameter-VJP pieces")
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
    if args.workload == "moe":
        workload_moe(args)
        return
    if args.workload == "pvjp":
        workload_pvjp(args)
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

    global GRAD_SQ_SLOTS
    GRAD_SQ_SLOTS = model.buffer("grad_sq_slots")[1]
    # live per-op timing: eager steps with a HIP event pair around every op
    # on the model stream, averaged over the profiled steps
    model.profile(True)
    for _ in range(max(1, args.profile_steps)):
        model.train_step(tc.learning_rate)
    prof = model.profile_collect()
    model.profile(False)
    nprof = max(1, args.profile_steps)
    prof = {op: (ms / nprof, calls // nprof) for op, (ms, calls) in prof.items()}
    # the same steps again with every GEMM op's kernel timed alone (events
    # its launch records at the kernel's own start and end)
    model.profile(True, kernels=True)
    for _ in range(nprof):
        model.train_step(tc.learning_rate)
    kprof = model.profile_collect()
    op_kernel = dict(model.profile_kernels)
    model.profile(False)
    kern_only = {op[:-len("#kernel")]: (ms / nprof, calls // nprof) for op, (ms, calls) in kprof.items()
                 if op.endswith("#kernel")}
    # and once more with the second stream running beside, as in the step:
    # each kernel's time while it shares the chip (the graph replay's case)
    model.profile(True, instep=True)
    for _ in range(nprof):
        model.train_step(tc.learning_rate)
    iprof = model.profile_collect()
    model.profile(False)
    kern_instep = {op[:-len("#kernel")]: (ms / nprof, calls // nprof) for op, (ms, calls) in iprof.items()
                   if op.endswith("#kernel")}
    # cold-cache pass: a 512 MiB buffer is written before every op, so the
    # bandwidth-bound ops read their operands from HBM rather than from the
    # 256 MB Infinity Cache
    cold = {}
    if args.cold_steps > 0:
        model.profile(True, cold=True)
        for _ in range(args.cold_steps):
            model.train_step(tc.learning_rate)
        cold = model.profile_collect()
        model.profile(False)
        cold = {op: (ms / args.cold_steps, calls // args.cold_steps) for op, (ms, calls) in cold.items()}
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
    cold_rows = {}
    for op, (ms, calls) in prof.items():
        kind, work = op_work(op, mc, tc)
        if kind != "byte" or op not in cold or work <= 0:
            continue
        hot_us, cold_us = ms * 1e3 / calls, cold[op][0] * 1e3 / max(cold[op][1], 1)
        cold_rows[op] = {"bytes": int(work), "hot_us": round(hot_us, 3), "cold_us": round(cold_us, 3),
                         "hot_gbs": round(work / (hot_us * 1e-6) / 1e9, 1),
                         "cold_gbs": round(work / (cold_us * 1e-6) / 1e9, 1),
                         "cold_frac": round(work / (cold_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
        extra = op_issued_bytes(op, mc, tc)
        if extra:  # what the kernel moves in all, beside the algorithmic bytes
            iss = work + extra
            cold_rows[op]["issued"] = {"bytes": int(iss), "cold_gbs": round(iss / (cold_us * 1e-6) / 1e9, 1),
                                       "cold_frac": round(iss / (cold_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    if cold_rows:
        # each op beside a plain copy of its own (issued) byte count under the
        # same protocol: the fraction of the copy's rate the op reaches
        sizes = {op: r.get("issued", r)["bytes"] for op, r in cold_rows.items()}
        ref = copy_reference(sorted(set(sizes.values())))
        for op, r in cold_rows.items():
            chot, ccold = ref[sizes[op]]
            r["copy_same_bytes"] = {"bytes": sizes[op], "hot_us": round(chot, 3), "cold_us": round(ccold, 3),
                                    "cold_gbs": round(sizes[op] / (ccold * 1e-6) / 1e9, 1)}
            r["hot_vs_copy"] = round(chot / r["hot_us"], 4)
            r["cold_vs_copy"] = round(ccold / r["cold_us"], 4)
        log("  bandwidth-bound ops, hot vs cold cache (512 MiB written before each op), "
            "and a plain copy of the op's issued bytes under the same protocol:")
        for op, r in sorted(cold_rows.items(), key=lambda kv: -kv[1]["bytes"]):
            c = r["copy_same_bytes"]
            log(f"  {op:24s} {r['bytes'] / 1e6:8.2f} MB  hot {r['hot_us']:8.2f} us {r['hot_gbs']:8.1f} GB/s  "
                f"cold {r['cold_us']:8.2f} us {r['cold_gbs']:8.1f} GB/s ({100 * r['cold_frac']:.1f}% of HBM)" +
                (f"; issued {r['issued']['bytes'] / 1e6:.2f} MB, {100 * r['issued']['cold_frac']:.1f}% cold"
                 if "issued" in r else "") +
                f"; copy hot {c['hot_us']:.2f} cold {c['cold_us']:.2f} us -> op at "
                f"{100 * r['hot_vs_copy']:.0f}% / {100 * r['cold_vs_copy']:.0f}% of the copy's rate")
    roofline = kernel_roofline(prof, kern_only, op_kernel, mc, tc, args.config, kern_instep)
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
        cpu = cpu_baseline(mc, tc, args.cpu_sample_batch or cpu_sample_batch(mc, tc))
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
        "data": "synthetic uniform random bytes (SplitMix64 seed 123), weights N(0,0.02) seed 42" +
                (", routers N(0,1/d) (logits N(0,1))" if getattr(mc, "experts", None) is not None else ""),
        "config": {"workload": (_hier_name(args.config, mc) if mc.hierarchy is not None else
                                f"{args.config}: {mc.layers}-layer MoE byte Transformer d{mc.width} GQA "
                                f"{mc.heads}/{mc.kv} hd{mc.head_dim}, {mc.experts.count} SwiGLU experts x "
                                f"{mc.experts.ffn_width} top-{mc.experts.top_k}, "
                                if getattr(mc, "experts", None) is not None else
                                f"{args.config}: {mc.layers}-layer byte Transformer d{mc.width} GQA "
                                f"{mc.heads}/{mc.kv} hd{mc.head_dim} SwiGLU {mc.ffn_width}, ") +
                               ("fwd+bwd+AdamW" if tc.optimizer == "adamw" else
                                "fwd+bwd+selected-row SGD" + (
                                    f" with rank-{tc.parameter_vjp.rank} parameter VJP, "
                                    f"{tc.parameter_vjp.residual_fraction:g} residual rows"
                                    if tc.parameter_vjp else "")),
                   "global_batch": tc.batch, "seq_len": tc.sequence, "tokens_per_step": tokens,
                   "parallelism": "single-gpu", "graph": not args.no_graph},
        "step_mfma": {"algorithmic_tflop_per_step": round(step_flops / 1e12, 4),
                      "achieved_tflops": round(step_tflops, 2), "frac": round(step_tflops / PEAK_BF16_TFLOPS, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cold_cache": cold_rows or None,
        "loss": loss,
    }
    print(json.dumps(out), flush=True)
    model.close()


if __name__ == "__main__":
    main()
