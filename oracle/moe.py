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


def _softmax64(logits):
    x = np.asarray(logits, np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def moe_forward(z, w_router, experts, top_k, dtype="bf16", logits=None):
    """z [M][d]; w_router [d][E]; experts = [(w_gate [d][F], w_up [d][F],
    w_down [F][d])].  dtype: storage rounding ("bf16", "f32" or None for
    exact: the expert choice still follows the fp32 rule, the weights and
    their backward are FP64).  `logits` (optional) conditions the routing on
    given stored logits.  Returns the activations the backward needs."""
    z = np.asarray(z, np.float64)
    M, d = z.shape
    E = len(experts)
    if logits is None:
        logits = _rnd(z @ w_router, dtype)
    ids, w = O.route_topk(np.asarray(logits, np.float32), top_k)
    if dtype is None:  # exact mode: the full-softmax weights of the chosen experts in FP64
        w = _softmax64(logits)[np.arange(M)[:, None], ids]
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
                slots=slots, per=per, update=_rnd(y, dtype), exact=dtype is None)


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
    if acts.get("exact"):  # route_topk_bwd's rule in FP64: p * (dy_selected - sum_k w_k dy_k)
        p = _softmax64(acts["logits"])
        sel = np.zeros_like(p)
        np.add.at(sel, (np.repeat(np.arange(M), ids.shape[1]), ids.ravel()), dweights.ravel())
        dlogits = p * (sel - np.sum(w * dweights, axis=1, keepdims=True))
    else:
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


# ------------------------------------------------------------------ model
# The MoE byte Transformer (ModelConfig::experts, crates/sejong-core/src/
# lib.rs:100-106): every block's FFN is the MoE branch of Block::apply
# (architecture.rs:229-242), the rest of the block, the final norm, the fp32
# head and the mean cross-entropy as the dense model (oracle.py
# body_forward / body_backward restated with that FFN).  cfg keys: d,
# layers, hq, hk, E (experts), K (top_k), fe (expert width), T, B, eps,
# theta.
#
# Pinning (tests/test_oracle.py): with E = 1 and K = 1 (every routing
# weight is exactly 1 and the router gradient exactly 0) the model equals
# the dense C oracle's with gate / up / down = expert 0's, forward and
# backward; the loss gradient against central finite differences in exact
# FP64 for entries of every tensor kind (routing held fixed).

def layout(cfg):
    """(name, shape) in the reference order (stage_layout,
    architecture.rs:63-95 with experts, then final_norm and output)."""
    d, E, fe = cfg["d"], cfg["E"], cfg["fe"]
    J = d // cfg["hq"] * cfg["hk"]
    out = [("embedding", (O.VOCAB, d))]
    for i in range(cfg["layers"]):
        p = f"layers.{i}"
        out += [(f"{p}.attention_norm", (d,)), (f"{p}.ffn_norm", (d,)), (f"{p}.query", (d, d)),
                (f"{p}.key", (d, J)), (f"{p}.value", (d, J)), (f"{p}.attention_output", (d, d))]
        for e in range(E):
            q = f"{p}.experts.{e}"
            out += [(f"{q}.gate", (d, fe)), (f"{q}.up", (d, fe)), (f"{q}.down", (fe, d))]
        out.append((f"{p}.router", (d, E)))
    return out + [("final_norm", (d,)), ("output", (d, O.VOCAB))]


def _offsets(cfg):
    off, table = 0, {}
    for name, shape in layout(cfg):
        table[name] = (off, shape)
        off += int(np.prod(shape))
    return table, off


def param_count(cfg):
    return _offsets(cfg)[1]


ACT_NAMES = ("x", "z", "qr", "kr", "v", "o", "lse", "x1", "z2", "rlog")


def acts_layout(cfg):
    """[(name, layer, size)] of the activation pack (sj_model_export_activations'
    order for the MoE model: the router's stored logits stand for g, u, h)."""
    d, L, hq, E = cfg["d"], cfg["layers"], cfg["hq"], cfg["E"]
    M, J = cfg["T"] * cfg["B"], d // hq * cfg["hk"]
    size = dict(x=M * d, z=M * d, qr=M * d, kr=M * J, v=M * J, o=M * d, lse=M * hq, x1=M * d, z2=M * d, rlog=M * E)
    out = [(n, l, size[n]) for l in range(L) for n in ACT_NAMES]
    return out + [("xL", -1, M * d), ("hn", -1, M * d), ("logits", -1, M * O.VOCAB)]


def unpack(cfg, flat):
    """{(name, layer): array} from a flat activation pack."""
    acts, off = {}, 0
    flat = np.asarray(flat, np.float64)
    for name, l, n in acts_layout(cfg):
        acts[(name, l)] = flat[off:off + n]
        off += n
    return acts


def _weights(cfg, params, dtype):
    table, _ = _offsets(cfg)
    params = np.asarray(params, np.float64)
    C = O.round_to(params, dtype) if dtype != "none" else params.copy()   # Model::bind compute copies

    def W(name, master=False):
        o, shape = table[name]
        return (params if master else C)[o:o + int(np.prod(shape))].reshape(shape)
    return table, W


def _experts(cfg, W, l):
    return [(W(f"layers.{l}.experts.{e}.gate"), W(f"layers.{l}.experts.{e}.up"), W(f"layers.{l}.experts.{e}.down"))
            for e in range(cfg["E"])]


def model_forward(cfg, params, ids, dtype="f32"):
    """The activation pack ({(name, layer): flat array}) of one forward."""
    table, W = _weights(cfg, params, dtype)
    d, L, hq, hk, T, B = cfg["d"], cfg["layers"], cfg["hq"], cfg["hk"], cfg["T"], cfg["B"]
    M, Dh = T * B, d // hq
    eps, theta = cfg.get("eps", 1e-6), cfg.get("theta", 10000.0)
    rd = (lambda v: O.round_to(v, dtype)) if dtype != "none" else (lambda v: np.asarray(v, np.float64))
    rf = (lambda v: O.round_to(v, "f32")) if dtype != "none" else (lambda v: np.asarray(v, np.float64))
    acts = {}
    x = W("embedding")[np.asarray(ids)]
    for l in range(L):
        p = f"layers.{l}"
        z = rd(O.rmsnorm_fwd(x, W(f"{p}.attention_norm"), eps))
        q, k, v = rd(O.matmul(z, W(f"{p}.query"))), rd(O.matmul(z, W(f"{p}.key"))), rd(O.matmul(z, W(f"{p}.value")))
        qr, kr = rd(O.rope(q, T, hq, Dh, theta)), rd(O.rope(k, T, hk, Dh, theta))
        o, lse = O.attention_fwd(qr, kr, v, B, T, hq, hk, Dh)
        o, lse = rd(o), rf(lse)
        x1 = rd(x + rd(O.matmul(o, W(f"{p}.attention_output"))))
        z2 = rd(O.rmsnorm_fwd(x1, W(f"{p}.ffn_norm"), eps))
        ma = moe_forward(z2, W(f"{p}.router"), _experts(cfg, W, l), cfg["K"], None if dtype == "none" else dtype)
        for name, val in (("x", x), ("z", z), ("qr", qr), ("kr", kr), ("v", v), ("o", o), ("lse", lse), ("x1", x1),
                          ("z2", z2), ("rlog", ma["logits"])):
            acts[(name, l)] = np.asarray(val, np.float64).ravel()
        x = rd(x1 + ma["update"])
    hn = rd(O.rmsnorm_fwd(x, W("final_norm"), eps))
    logits = rf(O.matmul(hn, W("output", master=True)))                 # fp32 head on the master
    acts[("xL", -1)], acts[("hn", -1)], acts[("logits", -1)] = x.ravel(), hn.ravel(), logits.ravel()
    return acts


def model_backward(cfg, params, acts, ids, targets, dtype="f32"):
    """(mean loss, reference-layout gradients, per-layer routing) from an
    activation pack: the expert FFNs are recomputed in FP64 from the stored
    z2 rows with the routing of the stored router logits."""
    table, W = _weights(cfg, params, dtype)
    d, L, hq, hk, T, B, E = cfg["d"], cfg["layers"], cfg["hq"], cfg["hk"], cfg["T"], cfg["B"], cfg["E"]
    M, Dh, J, V = T * B, d // hq, d // hq * hk, O.VOCAB
    eps, theta = cfg.get("eps", 1e-6), cfg.get("theta", 10000.0)
    _, total = _offsets(cfg)
    G = np.zeros(total)

    def put(name, g):
        o, shape = table[name]
        G[o:o + int(np.prod(shape))] += np.asarray(g, np.float64).ravel()

    def A(name, l, cols):
        return acts[(name, l)].reshape(M, cols)
    seed = float(np.float32(1.0) / np.float32(M))           # scale / count, graph.rs:539-549
    rows, dlog = O.cross_entropy(A("logits", -1, V), targets, seed)
    loss = float(np.mean(rows))
    put("output", O.matmul(A("hn", -1, d), dlog, ta=True))
    dh = O.matmul(dlog, W("output", master=True), tb=True)
    dres, dwf = O.rmsnorm_bwd(A("xL", -1, d), W("final_norm"), dh, eps)
    put("final_norm", dwf)
    routing = [None] * L
    for l in range(L - 1, -1, -1):
        p = f"layers.{l}"
        z2, experts = A("z2", l, d), _experts(cfg, W, l)
        ma = moe_forward(z2, W(f"{p}.router"), experts, cfg["K"], None if dtype == "none" else dtype,
                         logits=A("rlog", l, E))
        routing[l] = (ma["ids"], ma["w"], ma["counts"], ma["tokens"], ma["slots"])
        dz2, dwr, egr, _, _ = moe_backward(z2, W(f"{p}.router"), experts, ma, dres)
        put(f"{p}.router", dwr)
        for e, (dg, du, dd) in enumerate(egr):
            put(f"{p}.experts.{e}.gate", dg)
            put(f"{p}.experts.{e}.up", du)
            put(f"{p}.experts.{e}.down", dd)
        dx1, dfn = O.rmsnorm_bwd(A("x1", l, d), W(f"{p}.ffn_norm"), dz2, eps, dx_acc=dres)
        put(f"{p}.ffn_norm", dfn)
        o = A("o", l, d)
        dO = O.matmul(dx1, W(f"{p}.attention_output"), tb=True)
        put(f"{p}.attention_output", O.matmul(o, dx1, ta=True))
        dqr, dkr, dv, _ = O.attention_bwd(A("qr", l, d), A("kr", l, J), A("v", l, J), o, acts[("lse", l)], dO,
                                          B, T, hq, hk, Dh)
        dq, dk = O.rope(dqr, T, hq, Dh, theta, inverse=True), O.rope(dkr, T, hk, Dh, theta, inverse=True)
        z = A("z", l, d)
        dz = (O.matmul(dq, W(f"{p}.query"), tb=True) + O.matmul(dk, W(f"{p}.key"), tb=True)
              + O.matmul(dv, W(f"{p}.value"), tb=True))
        put(f"{p}.query", O.matmul(z, dq, ta=True))
        put(f"{p}.key", O.matmul(z, dk, ta=True))
        put(f"{p}.value", O.matmul(z, dv, ta=True))
        dres, dan = O.rmsnorm_bwd(A("x", l, d), W(f"{p}.attention_norm"), dz, eps, dx_acc=dx1)
        put(f"{p}.attention_norm", dan)
    put("embedding", O.embedding_bwd(dres, ids, V))
    return loss, G, routing


def model_loss(cfg, params, ids, targets, dtype="none"):
    acts = model_forward(cfg, params, ids, dtype)
    rows, _ = O.cross_entropy(acts[("logits", -1)].reshape(-1, O.VOCAB), targets, 1.0)
    return float(np.mean(rows))
