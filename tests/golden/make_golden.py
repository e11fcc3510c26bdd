"""Writes the golden fixtures in tests/golden/ from the pinned FP64 oracle.

    python -m tests.golden.make_golden          (from the repository root)

The reference cannot run in this image and ships no numeric fixtures for
this path (its known-answer programs are generative), so each fixture is the
oracle's answer on the reference's own closed-form inputs where it has them
(the attention values() case of crates/sejong-gpu/examples/
hierarchy_check.rs:11-15, the selection of parameter_vjp_check.rs:42-100)
and on seeded synthetic inputs otherwise.  tests/test_oracle.py regenerates
every fixture and compares (the oracle cannot drift); the GPU tests compare
the device against them.  Fixtures are .npz (no pickles)."""
from __future__ import annotations

import os

import numpy as np

from oracle import moe as OM
from oracle import oracle as O
from oracle import pvjp as OP

HERE = os.path.dirname(os.path.abspath(__file__))


def values(n, offset):
    """Closed-form inputs of crates/sejong-gpu/examples/hierarchy_check.rs:11-15."""
    return np.array([((i * 17 + offset) % 41 - 20.0) / 31.0 for i in range(n)], dtype=np.float32).astype(np.float64)


def cfg1_case():
    from sejong_amd.model import byte_batch, config, init_params, layout
    from sejong_amd.rng import Rng
    mc, tc = config("cfg1")
    params = init_params(mc, std=0.02, seed=42)
    ids, tg = byte_batch(Rng(123), tc.batch, tc.sequence)
    cfg = dict(d=mc.width, layers=mc.layers, hq=mc.heads, hk=mc.kv, ffn=mc.ffn_width, T=tc.sequence, B=tc.batch,
               eps=mc.norm_epsilon, theta=mc.rope_theta)
    loss, g, _, _ = O.model_fwd_bwd(cfg, params.astype(np.float64), ids, tg, dtype="f32")
    rng = np.random.default_rng(0)
    norms, idx = [], []
    off = 0
    for name, shape, _ in layout(mc):
        n = int(np.prod(shape))
        norms.append(np.linalg.norm(g[off:off + n]))
        idx.append(off + np.sort(rng.choice(n, min(n, 64), replace=False)))
        off += n
    idx = np.concatenate(idx)
    return dict(loss=np.array(loss), grad_norms=np.array(norms), sample_index=idx.astype(np.int64),
                sample_value=g[idx])


def attention_case():
    t, h, kh, d = 5, 4, 2, 4
    q, k, v, dy = values(t * h * d, 0), values(t * kh * d, 3), values(t * kh * d, 9), values(t * h * d, 12)
    out = dict(q=q, k=k, v=v, dy=dy)
    for window in (0, 3):
        o, lse = O.attention_fwd(q.reshape(t, h * d), k.reshape(t, kh * d), v.reshape(t, kh * d), 1, t, h, kh, d,
                                 window)
        dq, dk, dv, _ = O.attention_bwd(q.reshape(t, h * d), k.reshape(t, kh * d), v.reshape(t, kh * d), o, lse,
                                        dy.reshape(t, h * d), 1, t, h, kh, d, window)
        for name, val in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
            out[f"{name}_w{window}"] = np.asarray(val).ravel()
    return out


def router_case():
    rng = np.random.default_rng(3)
    R, E, K = 512, 8, 2
    logits = O.round_to(rng.normal(0, 1, (R, E)), "bf16")
    logits[:16, 2] = logits[:16, 6] = 3.0                         # exact ties: lowest index first
    ids, w = O.route_topk(logits.astype(np.float32), K)
    dy = rng.normal(0, 1, (R, K)).astype(np.float32).astype(np.float64)
    dx = O.route_topk_bwd(logits.astype(np.float32), ids, w, dy)
    tokens, slots, counts = O.route_pack(ids, E)
    return dict(logits=logits, ids=ids, weights=w, dy=dy, dlogits=dx, tokens=tokens, slots=slots, counts=counts)


def pvjp_case():
    seed_check = O.Rng(42).next_u64()                             # parameter_vjp_check.rs:61-66, prepare's draw
    c1, r1, m1 = OP.indices(seed_check, 71, 97, 5, 2, 33, 16)
    seed_cfg5 = O.Rng(124).next_u64()                             # cfg5 parameter-VJP seed 124
    # the first prepare of a cfg5 step is the last layer's gate/up group; its
    # donor is the up projection (widest member, last on ties: graph.rs:931-934)
    r, blocks, s = OP.budget(16, 0.1, 32, 16384, 1024, 2752)
    c5, r5, m5 = OP.indices(seed_cfg5, 1024, 2752, blocks, s, r, 32)
    return dict(seed_check=np.array(seed_check, np.uint64), check_columns=c1, check_rows=r1, check_map=m1,
                seed_cfg5=np.array(seed_cfg5, np.uint64), cfg5_columns=c5, cfg5_rows=r5, cfg5_map=m5,
                cfg5_budget=np.array([r, blocks, s]))


def moe_case():
    rng = np.random.default_rng(4)
    M, d, E, F, K = 48, 16, 4, 24, 2
    z = O.round_to(rng.normal(0, 1, (M, d)), "bf16")
    wr = O.round_to(rng.normal(0, d ** -0.5, (d, E)), "bf16")
    ex = [tuple(O.round_to(rng.normal(0, 0.2, s), "bf16") for s in ((d, F), (d, F), (F, d))) for _ in range(E)]
    acts = OM.moe_forward(z, wr, ex, K, dtype="bf16")
    dup = rng.normal(0, 1e-2, (M, d)).astype(np.float32).astype(np.float64)
    dz, dwr, grads, dw, dlog = OM.moe_backward(z, wr, ex, acts, dup)
    out = dict(z=z, wr=wr, dup=dup, ids=acts["ids"], weights=acts["w"], update=acts["update"], dz=dz, dwr=dwr,
               dweights=dw, dlogits=dlog)
    for e, (wg, wu, wd) in enumerate(ex):
        out[f"wg{e}"], out[f"wu{e}"], out[f"wd{e}"] = wg, wu, wd
        out[f"dwg{e}"], out[f"dwu{e}"], out[f"dwd{e}"] = grads[e]
    return out


CASES = {"cfg1_step": cfg1_case, "attention_values": attention_case, "router": router_case,
         "pvjp_selection": pvjp_case, "moe_ffn_tiny": moe_case}


def main():
    for name, fn in CASES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
