"""ctypes wrapper over the FP64 CPU oracle (oracle/sejong_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the sejong_amd product path.

Each wrapper takes/returns float64 numpy arrays and names the reference
formula it restates (the C file carries the file:line citations).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsejong_oracle.so")
VOCAB = 257

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_D = ctypes.POINTER(ctypes.c_double)
_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int32)
_U64 = ctypes.POINTER(ctypes.c_uint64)
_L = ctypes.c_long


def _declare(L):
    L.or_rng_next.argtypes = [_U64]; L.or_rng_next.restype = ctypes.c_uint64
    L.or_rng_index.argtypes = [_U64, ctypes.c_uint64]; L.or_rng_index.restype = ctypes.c_uint64
    L.or_rng_uniform.argtypes = [_U64]; L.or_rng_uniform.restype = ctypes.c_double
    L.or_rng_normal_fill.argtypes = [_U64, _D, _L, ctypes.c_double]
    L.or_round.argtypes = [_D, _L, ctypes.c_int]
    L.or_matmul.argtypes = [_D, _D, _D, _L, _L, _L, ctypes.c_int, ctypes.c_int]
    L.or_rmsnorm_fwd.argtypes = [_D, _D, _D, _L, _L, ctypes.c_double]
    L.or_rmsnorm_bwd.argtypes = [_D, _D, _D, _D, _D, _D, _L, _L, ctypes.c_double]
    L.or_rope.argtypes = [_D, _D, _L, _L, _L, _L, _L, ctypes.c_double, ctypes.c_int]
    L.or_attention_fwd.argtypes = [_D, _D, _D, _D, _D, _L, _L, _L, _L, _L, _L]
    L.or_attention_bwd.argtypes = [_D] * 10 + [_L] * 6
    L.or_swiglu_fwd.argtypes = [_D, _D, _D, _L]
    L.or_swiglu_bwd.argtypes = [_D, _D, _D, _D, _D, _L]
    L.or_embedding_fwd.argtypes = [_D, _I, _D, _L, _L]
    L.or_embedding_bwd.argtypes = [_D, _I, _D, _L, _L, _L]
    L.or_cross_entropy.argtypes = [_D, _I, _D, _D, _L, _L, ctypes.c_double]
    L.or_sum_squares.argtypes = [_D, _L]; L.or_sum_squares.restype = ctypes.c_double
    L.or_adamw.argtypes = [_D, _D, _D, _D, _L] + [ctypes.c_double] * 8
    L.or_route_topk.argtypes = [_F, _I, _D, _L, _L, _L]
    L.or_route_topk_bwd.argtypes = [_F, _I, _D, _D, _D, _L, _L, _L]
    L.or_route_pack.argtypes = [_I, _I, _I, _I, _L, _L, _L]
    L.or_model_param_count.argtypes = [_L] * 5; L.or_model_param_count.restype = _L
    L.or_model_acts_count.argtypes = [_L] * 7; L.or_model_acts_count.restype = _L
    L.or_model_forward.argtypes = [_L] * 7 + [ctypes.c_double] * 2 + [ctypes.c_int, _D, _I, _D]
    L.or_model_backward.argtypes = [_L] * 7 + [ctypes.c_double] * 2 + [ctypes.c_int, _D, _D, _I, _I, _D, _D]
    L.or_model_backward.restype = ctypes.c_double
    L.or_model_backward_dys.argtypes = [_L] * 7 + [ctypes.c_double] * 2 + [ctypes.c_int, _D, _D, _I, _I, _D, _D, _D]
    L.or_model_backward_dys.restype = ctypes.c_double
    L.or_model_backward_hidden.argtypes = [_L] * 7 + [ctypes.c_double] * 2 + [ctypes.c_int, _D, _D, _D, _D, _D]
    L.or_model_fwd_bwd.argtypes = [_L] * 7 + [ctypes.c_double] * 2 + [ctypes.c_int, _D, _I, _I, _D, _D, _D]
    L.or_model_fwd_bwd.restype = ctypes.c_double
    L.or_model_loss.argtypes = [_L] * 7 + [ctypes.c_double] * 2 + [ctypes.c_int, _D, _I, _I]
    L.or_model_loss.restype = ctypes.c_double
    L.or_stage_acts_count.argtypes = [_L] * 7; L.or_stage_acts_count.restype = _L
    L.or_stage_forward.argtypes = [_L] * 7 + [ctypes.c_double] * 2 + [ctypes.c_int, _L, _D, _D, _D]
    L.or_stage_backward.argtypes = [_L] * 7 + [ctypes.c_double] * 2 + [ctypes.c_int, _L, _D, _D, _D, _D, _D]
    L.or_num_threads.restype = ctypes.c_int


def _d(a):
    a = np.ascontiguousarray(a, dtype=np.float64)
    return a, a.ctypes.data_as(_D)


def _i(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(_I)


def _out(shape):
    a = np.zeros(shape, dtype=np.float64)
    return a, a.ctypes.data_as(_D)


DTYPE_CODE = {"f32": 0, "bf16": 4, "none": -1}


# ------------------------------------------------------------------ RNG
class Rng:
    """SplitMix64 `Rng` (crates/sejong-core/src/lib.rs:591-623)."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed)

    def next_u64(self) -> int:
        return lib().or_rng_next(ctypes.byref(self.state))

    def index(self, n: int) -> int:
        return lib().or_rng_index(ctypes.byref(self.state), n)

    def uniform(self) -> float:
        return lib().or_rng_uniform(ctypes.byref(self.state))

    def normal_fill(self, n: int, std: float) -> np.ndarray:
        out, p = _out(n)
        lib().or_rng_normal_fill(ctypes.byref(self.state), p, n, std)
        return out


# ----------------------------------------------------------- rounding
def round_to(x, dtype: str) -> np.ndarray:
    """Storage rounding of x to 'f32' / 'bf16' (RNE), returned as float64."""
    a = np.array(x, dtype=np.float64, copy=True)
    if DTYPE_CODE[dtype] >= 0:
        lib().or_round(a.ctypes.data_as(_D), a.size, DTYPE_CODE[dtype])
    return a


# ------------------------------------------------------------- ops
def matmul(A, B, ta=False, tb=False):
    A, pa = _d(A); B, pb = _d(B)
    M, K = (A.shape[1], A.shape[0]) if ta else A.shape
    N = B.shape[0] if tb else B.shape[1]
    C, pc = _out((M, N))
    lib().or_matmul(pa, pb, pc, M, N, K, int(ta), int(tb))
    return C


def rmsnorm_fwd(x, w, eps):
    x, px = _d(x); w, pw = _d(w)
    y, py = _out(x.shape)
    lib().or_rmsnorm_fwd(px, pw, py, x.shape[0], x.shape[1], eps)
    return y


def rmsnorm_bwd(x, w, dy, eps, dx_acc=None):
    x, px = _d(x); w, pw = _d(w); dy, pdy = _d(dy)
    pacc = None
    if dx_acc is not None:
        dx_acc, pacc = _d(dx_acc)
    dx, pdx = _out(x.shape); dw, pdw = _out(x.shape[1])
    lib().or_rmsnorm_bwd(px, pw, pdy, pacc, pdx, pdw, x.shape[0], x.shape[1], eps)
    return dx, dw


def rope(x, T, H, D, theta=10000.0, offset=0, inverse=False):
    x, px = _d(x)
    y, py = _out(x.shape)
    lib().or_rope(px, py, x.shape[0], T, H, D, offset, theta, int(inverse))
    return y


def attention_fwd(q, k, v, B, T, HQ, HK, D, window=0):
    q, pq = _d(q); k, pk = _d(k); v, pv = _d(v)
    o, po = _out(q.shape); lse, pl = _out(B * T * HQ)
    lib().or_attention_fwd(pq, pk, pv, po, pl, B, T, HQ, HK, D, window)
    return o, lse


def attention_bwd(q, k, v, o, lse, do, B, T, HQ, HK, D, window=0):
    q, pq = _d(q); k, pk = _d(k); v, pv = _d(v); o, po = _d(o); lse, pl = _d(lse); do, pdo = _d(do)
    dq, pdq = _out(q.shape); dk, pdk = _out(k.shape); dv, pdv = _out(v.shape); delta, pde = _out(B * T * HQ)
    lib().or_attention_bwd(pq, pk, pv, po, pl, pdo, pdq, pdk, pdv, pde, B, T, HQ, HK, D, window)
    return dq, dk, dv, delta


def swiglu_fwd(g, u):
    g, pg = _d(g); u, pu = _d(u)
    h, ph = _out(g.shape)
    lib().or_swiglu_fwd(pg, pu, ph, g.size)
    return h


def swiglu_bwd(g, u, dy):
    g, pg = _d(g); u, pu = _d(u); dy, pdy = _d(dy)
    dg, pdg = _out(g.shape); du, pdu = _out(g.shape)
    lib().or_swiglu_bwd(pg, pu, pdy, pdg, pdu, g.size)
    return dg, du


def embedding_fwd(W, ids):
    W, pw = _d(W); ids, pi = _i(ids)
    y, py = _out((ids.size, W.shape[1]))
    lib().or_embedding_fwd(pw, pi, py, ids.size, W.shape[1])
    return y


def embedding_bwd(dy, ids, V):
    dy, pdy = _d(dy); ids, pi = _i(ids)
    dW, pdw = _out((V, dy.shape[1]))
    lib().or_embedding_bwd(pdy, pi, pdw, ids.size, dy.shape[1], V)
    return dW


def cross_entropy(x, targets, dy_scale=1.0):
    x, px = _d(x); t, pt = _i(targets)
    loss, pl = _out(x.shape[0]); dx, pdx = _out(x.shape)
    lib().or_cross_entropy(px, pt, pl, pdx, x.shape[0], x.shape[1], dy_scale)
    return loss, dx


def sum_squares(g):
    g, pg = _d(g)
    return lib().or_sum_squares(pg, g.size)


def adamw(w, g, m, v, lr, b1, b2, eps, decay, ib1, ib2, scale):
    """Returns updated (w, m, v) as new arrays."""
    w, pw = _d(np.array(w, dtype=np.float64, copy=True)); g, pg = _d(g)
    m, pm = _d(np.array(m, dtype=np.float64, copy=True)); v, pv = _d(np.array(v, dtype=np.float64, copy=True))
    lib().or_adamw(pw, pg, pm, pv, w.size, lr, b1, b2, eps, decay, ib1, ib2, scale)
    return w, m, v


def route_topk(logits_f32, K):
    x = np.ascontiguousarray(logits_f32, dtype=np.float32)
    R, E = x.shape
    ids = np.zeros((R, K), dtype=np.int32); w, pw = _out((R, K))
    lib().or_route_topk(x.ctypes.data_as(_F), ids.ctypes.data_as(_I), pw, R, E, K)
    return ids, w


def route_topk_bwd(logits_f32, ids, weights, dy):
    x = np.ascontiguousarray(logits_f32, dtype=np.float32)
    R, E = x.shape
    K = ids.shape[1]
    ids, pi = _i(ids); weights, pw = _d(weights); dy, pdy = _d(dy)
    dx, pdx = _out((R, E))
    lib().or_route_topk_bwd(x.ctypes.data_as(_F), pi, pw, pdy, pdx, R, E, K)
    return dx


def route_pack(ids, E):
    ids, pi = _i(ids)
    S = ids.size
    K = ids.shape[1] if ids.ndim == 2 else 1
    tokens = np.full((E, S), -1, dtype=np.int32); slots = np.full((E, S), -1, dtype=np.int32)
    counts = np.zeros(E, dtype=np.int32)
    lib().or_route_pack(pi, tokens.ctypes.data_as(_I), slots.ctypes.data_as(_I), counts.ctypes.data_as(_I), S, K, E)
    return tokens, slots, counts


# -------------------------------------------------------------- model
def model_param_count(d, layers, hq, hk, ffn):
    return lib().or_model_param_count(d, layers, hq, hk, ffn)


def model_fwd_bwd(cfg, params, ids, targets, dtype="f32", want_logits=False):
    """Loss, gradients (reference layout, flat FP64) and optionally logits."""
    d, layers, hq, hk, ffn, T, B = (cfg["d"], cfg["layers"], cfg["hq"], cfg["hk"], cfg["ffn"], cfg["T"], cfg["B"])
    params, pp = _d(params)
    ids, pi = _i(ids); targets, pt = _i(targets)
    grads, pg = _out(params.size)
    rows, pr = _out(T * B)
    logits, plg = (_out((T * B, VOCAB)) if want_logits else (None, None))
    loss = lib().or_model_fwd_bwd(d, layers, hq, hk, ffn, T, B, cfg.get("eps", 1e-6), cfg.get("theta", 10000.0),
                                  DTYPE_CODE[dtype], pp, pi, pt, pg, pr, plg)
    return loss, grads, rows, logits


def _dims(cfg):
    return (cfg["d"], cfg["layers"], cfg["hq"], cfg["hk"], cfg["ffn"], cfg["T"], cfg["B"])


def model_acts_count(cfg):
    return lib().or_model_acts_count(*_dims(cfg))


def model_forward(cfg, params, ids, dtype="f32"):
    """Activation pack (see or_model_acts_count) of the forward pass."""
    params, pp = _d(params); ids, pi = _i(ids)
    acts, pa = _out(model_acts_count(cfg))
    lib().or_model_forward(*_dims(cfg), cfg.get("eps", 1e-6), cfg.get("theta", 10000.0), DTYPE_CODE[dtype],
                           pp, pi, pa)
    return acts


def model_backward(cfg, params, acts, ids, targets, dtype="f32", want_dys=False):
    """Loss, reference-layout gradients and per-row losses from an
    activation pack (e.g. the device's stored activations).  want_dys adds
    a list with, per layer, the output gradients of the projection Matmul
    nodes {"q", "k", "v" (pre-RoPE), "gate", "up"}."""
    params, pp = _d(params); acts, pa = _d(acts); ids, pi = _i(ids); targets, pt = _i(targets)
    grads, pg = _out(params.size); rows, pr = _out(cfg["T"] * cfg["B"])
    d, L, hq, hk, F, T, B = _dims(cfg)
    M, J = T * B, d // hq * hk
    if not want_dys:
        loss = lib().or_model_backward(*_dims(cfg), cfg.get("eps", 1e-6), cfg.get("theta", 10000.0),
                                       DTYPE_CODE[dtype], pp, pa, pi, pt, pg, pr)
        return loss, grads, rows
    dys, py = _out(L * M * (d + 2 * J + 2 * F))
    loss = lib().or_model_backward_dys(*_dims(cfg), cfg.get("eps", 1e-6), cfg.get("theta", 10000.0),
                                       DTYPE_CODE[dtype], pp, pa, pi, pt, pg, pr, py)
    per, off = [], 0
    for _ in range(L):
        layer = {}
        for name, width in (("q", d), ("k", J), ("v", J), ("gate", F), ("up", F)):
            layer[name] = dys[off:off + M * width].reshape(M, width)
            off += M * width
        per.append(layer)
    return loss, grads, rows, per


def model_backward_hidden(cfg, params, acts, dh, dtype="f32"):
    """The body's backward from d(final-norm output) dh [M][d] (another head
    on the body): reference-layout gradients (embedding / output zero) and the
    gradient at the embedding output [M][d].  acts may stop before the
    logits."""
    params, pp = _d(params); dh, pd = _d(dh)
    a = np.zeros(model_acts_count(cfg))
    acts = np.asarray(acts, np.float64).ravel()
    a[:acts.size] = acts
    a, pa = _d(a)
    grads, pg = _out(params.size)
    d, L, hq, hk, F, T, B = _dims(cfg)
    demb, pe = _out((T * B, d))
    lib().or_model_backward_hidden(*_dims(cfg), cfg.get("eps", 1e-6), cfg.get("theta", 10000.0), DTYPE_CODE[dtype],
                                   pp, pa, pd, pg, pe)
    return grads, demb


def acts_layout(cfg):
    """[(name, layer, size)] of the activation pack, in order."""
    d, L, hq, hk, F, T, B = _dims(cfg)
    M, J = T * B, d // hq * hk
    out = []
    for l in range(L):
        out += [("x", l, M * d), ("z", l, M * d), ("qr", l, M * d), ("kr", l, M * J), ("v", l, M * J),
                ("o", l, M * d), ("lse", l, M * hq), ("x1", l, M * d), ("z2", l, M * d), ("g", l, M * F),
                ("u", l, M * F), ("h", l, M * F)]
    out += [("xL", -1, M * d), ("hn", -1, M * d), ("logits", -1, M * VOCAB)]
    return out


def stage_acts_count(cfg):
    return lib().or_stage_acts_count(*_dims(cfg))


def stage_forward(cfg, sparams, x_in, dtype="f32"):
    """One stage of the hierarchical model (or_stage_forward): cfg as the
    model's plus "window"; sparams = the stage's tensors in stage_layout
    order then its closing norm; x_in [M][d].  Returns the stage's
    activation pack (per layer as acts_layout, then the last residual and
    the closing norm's output)."""
    sparams, pp = _d(sparams); x_in, px = _d(x_in)
    acts, pa = _out(stage_acts_count(cfg))
    lib().or_stage_forward(*_dims(cfg), cfg.get("eps", 1e-6), cfg.get("theta", 10000.0), DTYPE_CODE[dtype],
                           cfg.get("window", 0), pp, px, pa)
    return acts


def stage_backward(cfg, sparams, acts, dz, dtype="f32"):
    """(gradients in the sparams layout, d(stage input)) from d(closing
    norm output) dz [M][d]."""
    sparams, pp = _d(sparams); acts, pa = _d(acts); dz, pd = _d(dz)
    grads, pg = _out(sparams.size)
    dx, pdx = _out((cfg["T"] * cfg["B"], cfg["d"]))
    lib().or_stage_backward(*_dims(cfg), cfg.get("eps", 1e-6), cfg.get("theta", 10000.0), DTYPE_CODE[dtype],
                            cfg.get("window", 0), pp, pa, pd, pg, pdx)
    return grads, dx


def model_loss(cfg, params, ids, targets, dtype="f32"):
    d, layers, hq, hk, ffn, T, B = (cfg["d"], cfg["layers"], cfg["hq"], cfg["hk"], cfg["ffn"], cfg["T"], cfg["B"])
    params, pp = _d(params)
    ids, pi = _i(ids); targets, pt = _i(targets)
    return lib().or_model_loss(d, layers, hq, hk, ffn, T, B, cfg.get("eps", 1e-6), cfg.get("theta", 10000.0),
                               DTYPE_CODE[dtype], pp, pi, pt)


def num_threads():
    return lib().or_num_threads()
