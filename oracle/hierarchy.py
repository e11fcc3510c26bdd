"""Restatement of the hierarchical model's patch maps (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may import
this module; the product path never does.

The reference kernels (python/sejong_kernels/ops/hierarchy.py:107-172,
launched by crates/sejong-gpu/src/hierarchy_ops.rs:149-278) form their sums
in fp32, one position after another; this restatement does the same in
numpy float32 (elementwise IEEE single operations in the same order), so
the device must match it bit for bit.  Inputs in a bf16 storage dtype are
given as their exact values.

Pinning (tests/test_oracle.py): closed forms (the mean of constant and
linear patches, a partial last patch, patch longer than the sequence, the
shift by one patch with the BOS row first) and the adjoint identities
<pool(x), y> = <x, pool_backward(y)> and <broadcast(x, bos), dy> =
<x, dx> + <bos, dbos>, which fix the backward maps from the forward ones.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


def _store(v, dtype):
    return O.round_to(np.asarray(v, np.float64), dtype) if dtype == "bf16" else np.asarray(v, np.float32).astype(np.float64)


def patch_pool(x, batch, t, patch, dtype="f32"):
    """hierarchy.py:107-119: y[row] = (sum of the patch's rows in order) / count."""
    x = np.asarray(x, np.float32).reshape(batch, t, -1)
    d = x.shape[2]
    patches = -(-t // patch)
    y = np.zeros((batch, patches, d), np.float32)
    for p in range(patches):
        start = p * patch
        count = min(patch, t - start)
        total = np.zeros((batch, d), np.float32)
        for q in range(count):
            total = total + x[:, start + q]
        y[:, p] = total / np.float32(count)
    return _store(y.reshape(batch * patches, d), dtype)


def patch_pool_backward(dy, batch, t, patch):
    """hierarchy.py:122-131: dx[b, pos] = dy[b, pos // patch] / count (fp32)."""
    dy = np.asarray(dy, np.float32)
    d = dy.shape[-1]
    patches = -(-t // patch)
    dy = dy.reshape(batch, patches, d)
    dx = np.zeros((batch, t, d), np.float32)
    for pos in range(t):
        p = pos // patch
        count = min(patch, t - p * patch)
        dx[:, pos] = dy[:, p] / np.float32(count)
    return dx.reshape(batch * t, d).astype(np.float64)


def patch_broadcast(x, bos, batch, t, patch):
    """hierarchy.py:134-143: y[b, pos] = x[b, pos // patch - 1], bos for the first patch."""
    x = np.asarray(x, np.float64)
    d = x.shape[-1]
    patches = -(-t // patch)
    x = x.reshape(batch, patches, d)
    y = np.zeros((batch, t, d))
    for pos in range(t):
        p = pos // patch - 1
        y[:, pos] = x[:, p] if p >= 0 else np.asarray(bos, np.float64).reshape(d)
    return y.reshape(batch * t, d)


def patch_broadcast_backward(dy, batch, t, patch):
    """hierarchy.py:146-172: dx[b, p] = sum over offsets of dy[b, (p+1)*patch
    + offset] (masked positions add 0); dbos = sum over batches, then over the
    first patch's positions; fp32 in that order."""
    dy = np.asarray(dy, np.float32)
    d = dy.shape[-1]
    dy = dy.reshape(batch, t, d)
    patches = -(-t // patch)
    dx = np.zeros((batch, patches, d), np.float32)
    for p in range(patches):
        total = np.zeros((batch, d), np.float32)
        for off in range(patch):
            pos = (p + 1) * patch + off
            total = total + (dy[:, pos] if pos < t else np.float32(0.0))
        dx[:, p] = total
    dbos = np.zeros(d, np.float32)
    for b in range(batch):
        for pos in range(min(patch, t)):
            dbos = dbos + dy[b, pos]
    return dx.reshape(batch * patches, d).astype(np.float64), dbos.astype(np.float64)


# ------------------------------------------------------ hierarchical model
# hidden_from_encoded (crates/sejong-model/src/architecture.rs:368-393) with
# encode (:317-345) and the output head (lib.rs:336-340), in FP64 with the
# reference's storage roundings (every Graph::matmul / add / patch op stores
# in the compute dtype, graph.rs:203-221), and its reverse by the tape's
# rules (graph.rs:567-911).  cfg keys: the global stage as for the dense
# model (d, layers, hq, hk, ffn), T (bytes per sequence), B, eps, theta and
# P (patch size), window (local), encoder de / le / he / fe and decoder
# dd / ld / hd / fd (width, layers, heads = kv heads, FFN width).
#
# Pinning (tests/test_oracle.py): the loss gradient against central finite
# differences of the loss in exact FP64 for tensors of every stage and of
# every glue projection, and with the local stages' window wider than the
# sequence the hierarchical stages reduce to the dense oracle's blocks.


def layout(cfg):
    """(name, shape) in the reference order (architecture.rs:96-137)."""
    V = O.VOCAB

    def stage(prefix, d, L, hq, hk, F):
        J = d // hq * hk
        out = []
        for i in range(L):
            p = f"{prefix}.{i}"
            out += [(f"{p}.attention_norm", (d,)), (f"{p}.ffn_norm", (d,)), (f"{p}.query", (d, d)),
                    (f"{p}.key", (d, J)), (f"{p}.value", (d, J)), (f"{p}.attention_output", (d, d)),
                    (f"{p}.gate", (d, F)), (f"{p}.up", (d, F)), (f"{p}.down", (F, d))]
        return out
    d, de, dd = cfg["d"], cfg["de"], cfg["dd"]
    return ([("embedding", (V, de))] + stage("encoder", de, cfg["le"], cfg["he"], cfg["he"], cfg["fe"])
            + [("encoder_norm", (de,)), ("input_projection", (d, de)), ("encoder_to_global", (de, d)),
               ("encoder_to_decoder", (de, dd)), ("global_to_decoder", (d, dd)), ("global_bos", (1, d)),
               ("global_norm", (d,))]
            + stage("layers", d, cfg["layers"], cfg["hq"], cfg["hk"], cfg["ffn"])
            + stage("decoder", dd, cfg["ld"], cfg["hd"], cfg["hd"], cfg["fd"])
            + [("decoder_norm", (dd,)), ("output_projection", (dd, d)), ("final_norm", (d,)), ("output", (d, V))])


def _offsets(cfg):
    off, table = 0, {}
    for name, shape in layout(cfg):
        n = int(np.prod(shape))
        table[name] = (off, shape)
        off += n
    return table, off


def param_count(cfg):
    return _offsets(cfg)[1]


def _stage_cfgs(cfg):
    Tg = -(-cfg["T"] // cfg["P"])
    base = dict(B=cfg["B"], eps=cfg.get("eps", 1e-6), theta=cfg.get("theta", 10000.0))
    w = cfg["window"]
    return {"encoder": dict(base, d=cfg["de"], layers=cfg["le"], hq=cfg["he"], hk=cfg["he"], ffn=cfg["fe"],
                            T=cfg["T"], window=w if w < cfg["T"] else 0),
            "layers": dict(base, d=cfg["d"], layers=cfg["layers"], hq=cfg["hq"], hk=cfg["hk"], ffn=cfg["ffn"],
                           T=Tg, window=0),
            "decoder": dict(base, d=cfg["dd"], layers=cfg["ld"], hq=cfg["hd"], hk=cfg["hd"], ffn=cfg["fd"],
                            T=cfg["T"], window=w if w < cfg["T"] else 0)}


_NORM = {"encoder": "encoder_norm", "layers": "global_norm", "decoder": "decoder_norm"}


def _stage_slice(cfg, table, prefix):
    """Offsets of the stage's tensors (stage_layout order) and its closing norm."""
    L = {"encoder": cfg["le"], "layers": cfg["layers"], "decoder": cfg["ld"]}[prefix]
    names = [f"{prefix}.{i}.{t}" for i in range(L) for t in ("attention_norm", "ffn_norm", "query", "key", "value",
                                                              "attention_output", "gate", "up", "down")]
    return names + [_NORM[prefix]]


def _gather(params, table, names):
    return np.concatenate([params[table[n][0]:table[n][0] + int(np.prod(table[n][1]))] for n in names])


def _scatter(grads, table, names, flat):
    off = 0
    for n in names:
        o, shape = table[n]
        k = int(np.prod(shape))
        grads[o:o + k] += flat[off:off + k]
        off += k


def acts_layout(cfg):
    """[(name, size)] of the activation pack (sj_model_export_activations'
    order for the hierarchical model)."""
    sc = _stage_cfgs(cfg)
    out = [(f"stage:{k}", O.stage_acts_count(sc[k])) for k in ("encoder", "layers", "decoder")]
    Ml, Mg = cfg["B"] * cfg["T"], cfg["B"] * sc["layers"]["T"]
    de, d, dd = cfg["de"], cfg["d"], cfg["dd"]
    out += [("pooled", Mg * de), ("gd", Mg * dd), ("bosd", dd), ("zb", Ml * dd), ("bytes", Ml * dd),
            ("opo", Ml * d), ("hn", Ml * d), ("logits", Ml * O.VOCAB)]
    return out


def unpack(cfg, flat):
    acts, off = {}, 0
    for name, n in acts_layout(cfg):
        acts[name] = np.asarray(flat[off:off + n], np.float64)
        off += n
    return acts


def model_forward(cfg, params, ids, dtype="f32"):
    """The activation pack (dict keyed as acts_layout) of one forward."""
    table, _ = _offsets(cfg)
    sc = _stage_cfgs(cfg)
    params = np.asarray(params, np.float64)
    C = O.round_to(params, dtype) if dtype != "none" else params.copy()   # Model::bind compute copies

    def W(name):
        o, shape = table[name]
        return C[o:o + int(np.prod(shape))].reshape(shape)
    B, T, P = cfg["B"], cfg["T"], cfg["P"]
    Ml, Mg = B * T, B * sc["layers"]["T"]
    de, d, dd = cfg["de"], cfg["d"], cfg["dd"]
    rd = (lambda v: O.round_to(v, dtype)) if dtype != "none" else (lambda v: np.asarray(v, np.float64))
    acts = {}
    x0 = W("embedding")[np.asarray(ids)]
    acts["stage:encoder"] = O.stage_forward(sc["encoder"], _gather(C, table, _stage_slice(cfg, table, "encoder")),
                                            x0, dtype)
    en = acts["stage:encoder"][-Ml * de:].reshape(Ml, de)
    pooled = (patch_pool(en, B, T, P, dtype) if dtype != "none" else _pool64(en, B, T, P))
    acts["pooled"] = pooled.ravel()
    xg0 = rd(O.matmul(pooled.reshape(Mg, de), W("encoder_to_global")))
    acts["stage:layers"] = O.stage_forward(sc["layers"], _gather(C, table, _stage_slice(cfg, table, "layers")),
                                           xg0, dtype)
    gn = acts["stage:layers"][-Mg * d:].reshape(Mg, d)
    gd = rd(O.matmul(gn, W("global_to_decoder")))
    bosd = rd(O.matmul(W("global_bos"), W("global_to_decoder")))
    zb = patch_broadcast(gd, bosd, B, T, P)
    byt = rd(O.matmul(en, W("encoder_to_decoder")))
    xd0 = rd(byt + zb)
    acts.update(gd=gd.ravel(), bosd=bosd.ravel(), zb=zb.ravel(), bytes=byt.ravel())
    acts["stage:decoder"] = O.stage_forward(sc["decoder"], _gather(C, table, _stage_slice(cfg, table, "decoder")),
                                            xd0, dtype)
    dn = acts["stage:decoder"][-Ml * dd:].reshape(Ml, dd)
    opo = rd(O.matmul(dn, W("output_projection")))
    hn = rd(O.rmsnorm_fwd(opo, W("final_norm"), cfg.get("eps", 1e-6)))
    o, shape = table["output"]
    logits = O.matmul(hn, params[o:o + d * O.VOCAB].reshape(d, O.VOCAB))   # fp32 head on the master
    logits = O.round_to(logits, "f32") if dtype != "none" else logits
    acts.update(opo=opo.ravel(), hn=hn.ravel(), logits=logits.ravel())
    return acts


def _pool64(x, batch, t, patch):
    x = np.asarray(x, np.float64).reshape(batch, t, -1)
    patches = -(-t // patch)
    return np.stack([x[:, p * patch:min(t, (p + 1) * patch)].mean(1) for p in range(patches)], 1).reshape(
        batch * patches, -1)


def model_backward(cfg, params, acts, ids, targets, dtype="f32"):
    """(mean loss, reference-layout gradients) from an activation pack."""
    table, total = _offsets(cfg)
    sc = _stage_cfgs(cfg)
    params = np.asarray(params, np.float64)
    C = O.round_to(params, dtype) if dtype != "none" else params.copy()

    def W(name):
        o, shape = table[name]
        return C[o:o + int(np.prod(shape))].reshape(shape)
    B, T, P = cfg["B"], cfg["T"], cfg["P"]
    Ml, Mg = B * T, B * sc["layers"]["T"]
    de, d, dd, V = cfg["de"], cfg["d"], cfg["dd"], O.VOCAB
    eps = cfg.get("eps", 1e-6)
    G = np.zeros(total)

    def put(name, g):
        o, shape = table[name]
        G[o:o + int(np.prod(shape))] += np.asarray(g, np.float64).ravel()
    logits = acts["logits"].reshape(Ml, V)
    seed = float(np.float32(1.0) / np.float32(Ml))           # scale / count, graph.rs:539-549
    rows, dlog = O.cross_entropy(logits, targets, seed)
    loss = float(np.mean(rows))
    hn = acts["hn"].reshape(Ml, d)
    o, _ = table["output"]
    put("output", O.matmul(hn, dlog, ta=True))
    dh = O.matmul(dlog, params[o:o + d * V].reshape(d, V), tb=True)
    opo = acts["opo"].reshape(Ml, d)
    dopo, dwf = O.rmsnorm_bwd(opo, W("final_norm"), dh, eps)
    put("final_norm", dwf)
    dn = acts["stage:decoder"][-Ml * dd:].reshape(Ml, dd)
    put("output_projection", O.matmul(dn, dopo, ta=True))
    ddn = O.matmul(dopo, W("output_projection"), tb=True)
    names = _stage_slice(cfg, table, "decoder")
    g, dxd = O.stage_backward(sc["decoder"], _gather(C, table, names), acts["stage:decoder"], ddn, dtype)
    _scatter(G, table, names, g)
    en = acts["stage:encoder"][-Ml * de:].reshape(Ml, de)
    put("encoder_to_decoder", O.matmul(en, dxd, ta=True))
    den = O.matmul(dxd, W("encoder_to_decoder"), tb=True)
    dgd, dbos = patch_broadcast_backward(dxd, B, T, P)
    gn = acts["stage:layers"][-Mg * d:].reshape(Mg, d)
    put("global_to_decoder", O.matmul(gn, dgd, ta=True) + O.matmul(W("global_bos"), dbos.reshape(1, dd), ta=True))
    put("global_bos", O.matmul(dbos.reshape(1, dd), W("global_to_decoder"), tb=True))
    dgn = O.matmul(dgd, W("global_to_decoder"), tb=True)
    names = _stage_slice(cfg, table, "layers")
    g, dxg = O.stage_backward(sc["layers"], _gather(C, table, names), acts["stage:layers"], dgn, dtype)
    _scatter(G, table, names, g)
    pooled = acts["pooled"].reshape(Mg, de)
    put("encoder_to_global", O.matmul(pooled, dxg, ta=True))
    dpool = O.matmul(dxg, W("encoder_to_global"), tb=True)
    den = den + patch_pool_backward(dpool, B, T, P)
    names = _stage_slice(cfg, table, "encoder")
    g, dx0 = O.stage_backward(sc["encoder"], _gather(C, table, names), acts["stage:encoder"], den, dtype)
    _scatter(G, table, names, g)
    put("embedding", O.embedding_bwd(dx0, ids, V))
    return loss, G


def model_loss(cfg, params, ids, targets, dtype="none"):
    acts = model_forward(cfg, params, ids, dtype)
    rows, _ = O.cross_entropy(acts["logits"].reshape(-1, O.VOCAB), targets, 1.0)
    return float(np.mean(rows))
