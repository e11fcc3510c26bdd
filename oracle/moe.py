"""FP64 restatement of the mixture-of-experts FFN (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may import
this module; the product path never does.

Forward follows Block::apply's MoE branch (crates/sejong-model/src/
architecture.rs:229-242): router logits = z W_router stored in the compute
dtype (Graph::matmul, crates/sejong-gpu/src/graph.rs:212-220), top-k routing
(hierarchy.py:175-191, the C oracle's or_route_topk), the stable pack of
expert_routes (hierarchy.py:212-225, or_route_pack), per expert gather +
Ffn::apply (gate/up rounded to the storage dtype, SwiGLU from the rounded
values, down; architecture.rs:175-184, projection.py:67-73), and
expert_combine (hierarchy.py:228-235: y[token] += w[slot] * x, experts in
ascending order) cast to the compute dtype (hierarchy_ops.rs:413).

Backward follows the tape's rules (graph.rs:600-624, 749-754, 829-878):
combine backward (hierarchy.py:238-251), the experts' FFN backward, the
gather's scatter-add, route_topk backward (hierarchy.py:194-209) and the
router matmul's dX / dW.  All arithmetic is float64.

Pinning (tests/test_oracle.py): finite differences of a scalar projection of
the output with respect to every input on tiny shapes (routing held fixed),
and the E = 1, K = 1 special case, which is exactly the dense FFN.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


def _rnd(x, dtype):
    return O.round_to(x, dtype) if dtype else np.asarray(x, np.float64)


def moe_forward(z, w_router, experts, top_k, dtype="bf16", logits=None):
    """z [M][d]; w_router [d][E]; experts = [(w_gate [d][F], w_up [d][F],
    w_down [F][d])].  dtype: storage rounding ("bf16", "f32" or None for
    exact).  `logits` (optional) conditions the routing on given stored
    logits.  Returns the activations the backward needs."""
    z = np.asarray(z, np.float64)
    M, d = z.shape
    E = len(experts)
    if logits is None:
        logits = _rnd(z @ w_router, dtype)
    ids, w = O.route_topk(np.asarray(logits, np.float32), top_k)
    tokens, slots, counts = O.route_pack(ids, E)
    wflat = w.ravel()
    y = np.zeros((M, d))
    per = []
    for e, (wg, wu, wd) in enumerate(experts):
        c = int(counts[e])
        tk, sl = tokens[e, :c].astype(np.int64), slots[e, :c].astype(np.int64)
        x = z[tk]
        g = _rnd(x @ wg, dtype)
        u = _rnd(x @ wu, dtype)
        h = _rnd(O.swiglu_fwd(g, u), dtype)
        ye = _rnd(h @ wd, dtype)
        np.add.at(y, tk, wflat[sl][:, None] * ye)
        per.append(dict(tokens=tk, slots=sl, x=x, g=g, u=u, h=h, y=ye))
    return dict(logits=np.asarray(logits, np.float64), ids=ids, w=w, counts=counts, tokens=tokens,
                slots=slots, per=per, update=_rnd(y, dtype))


def moe_backward(z, w_router, experts, acts, dupdate):
    """Gradients of the MoE FFN given d(update) [M][d].  Returns dz,
    dW_router, [(dW_gate, dW_up, dW_down)], d(weights) [M][K], dlogits."""
    z = np.asarray(z, np.float64)
    dupdate = np.asarray(dupdate, np.float64)
    M, d = z.shape
    ids, w = acts["ids"], acts["w"]
    wflat = w.ravel()
    dweights = np.zeros(wflat.size)
    dz = np.zeros((M, d))
    grads = []
    for (wg, wu, wd), a in zip(experts, acts["per"]):
        tk, sl = a["tokens"], a["slots"]
        dy = dupdate[tk]
        dx = dy * wflat[sl][:, None]
        dweights[sl] = np.sum(a["y"] * dy, axis=1)
        dh = dx @ wd.T
        dg, du = O.swiglu_bwd(a["g"], a["u"], dh)
        grads.append((a["x"].T @ dg, a["x"].T @ du, a["h"].T @ dx))
        np.add.at(dz, tk, dg @ wg.T + du @ wu.T)
    dweights = dweights.reshape(ids.shape)
    dlogits = O.route_topk_bwd(np.asarray(acts["logits"], np.float32), ids, w, dweights)
    dz += dlogits @ np.asarray(w_router, np.float64).T
    dwr = z.T @ dlogits
    return dz, dwr, grads, dweights, dlogits


def dense_ffn(z, wg, wu, wd, dtype="bf16"):
    """Ffn::apply of a dense layer (architecture.rs:175-184), for the E = 1
    special case."""
    g = _rnd(z @ wg, dtype)
    u = _rnd(z @ wu, dtype)
    h = _rnd(O.swiglu_fwd(g, u), dtype)
    return _rnd(h @ wd, dtype)
