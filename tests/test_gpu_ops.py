"""Per-op parity of the HIP kernels against the FP64 oracle on identical
(storage-rounded) inputs.  Every call goes through the C ABI."""
import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_stored_close, dev, host, p, rel, rnd, sync, torch

pytestmark = pytest.mark.gpu

BF, F32 = 4, 0
DT = {"bf16": BF, "f32": F32}


@pytest.fixture(scope="module")
def api():
    from sejong_amd import _native as N
    N.load()
    return N.api


def ws(nbytes):
    t = torch()
    return t.empty(max(int(nbytes), 256), dtype=t.uint8, device="cuda")


# ------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("dt,R,D", [("bf16", 1000, 384), ("f32", 256, 128), ("bf16", 33, 1024)])
def test_rmsnorm_forward_backward(api, dt, R, D):
    rng = np.random.default_rng(1)
    x = rnd((R, D), dt, rng); w = rnd(D, dt, rng); dy = rng.normal(0, 1e-3, (R, D)).astype(np.float32).astype(np.float64)
    acc = rng.normal(0, 1e-3, (R, D)).astype(np.float32).astype(np.float64)
    eps = 1e-6
    X, W, DY, ACC = dev(x, dt), dev(w, dt), dev(dy), dev(acc)
    Y = torch().empty((R, D), dtype=X.dtype, device="cuda")
    api.sj_rmsnorm_fwd(None, p(X), DT[dt], p(W), DT[dt], p(Y), R, D, ctypes.c_float(eps))
    DX = torch().empty((R, D), device="cuda"); DWt = torch().empty(D, device="cuda")
    from sejong_amd import _native as N
    wsb = ws(N.load().sj_rmsnorm_bwd_workspace_bytes(R, D))
    api.sj_rmsnorm_bwd(None, p(X), DT[dt], p(W), DT[dt], p(DY), p(ACC), p(DX), p(DWt), R, D, ctypes.c_float(eps), p(wsb), wsb.numel())
    sync()
    assert_stored_close(host(Y), O.rmsnorm_fwd(x, w, eps), dt, "rmsnorm y")
    dx, dw = O.rmsnorm_bwd(x, w, dy, eps, dx_acc=acc)
    assert rel(host(DX), dx) < 1e-5 and rel(host(DWt), dw) < 1e-5


# ---------------------------------------------------------------- GEMM
GEMM_CASES = [
    # M, N, K, ta, tb, adt, bdt, cdt
    (256, 384, 384, 0, 0, "bf16", "bf16", "f32"),
    (4096, 640, 384, 0, 0, "bf16", "bf16", "bf16"),
    (333, 257, 190, 0, 0, "bf16", "f32", "f32"),   # head fwd: odd N / ld
    (4096, 384, 640, 0, 1, "f32", "bf16", "f32"),  # dX = dY W^T
    (512, 384, 257, 0, 1, "f32", "f32", "f32"),    # head dX
    (384, 640, 4096, 1, 0, "bf16", "f32", "f32"),  # dW, split-K
    (384, 257, 1000, 1, 0, "bf16", "f32", "f32"),  # head dW, edges
    (100, 70, 90, 1, 1, "f32", "f32", "f32"),
    (128, 96, 64, 1, 1, "bf16", "bf16", "f32"),
]


@pytest.mark.parametrize("M,N,K,ta,tb,adt,bdt,cdt", GEMM_CASES)
def test_gemm(api, M, N, K, ta, tb, adt, bdt, cdt):
    rng = np.random.default_rng(M + N + K)
    A = rnd((K, M) if ta else (M, K), adt, rng)
    B = rnd((N, K) if tb else (K, N), bdt, rng)
    ref = O.matmul(A, B, ta, tb)
    dA, dB = dev(A, adt), dev(B, bdt)
    C = torch().zeros((M, N), dtype=torch().bfloat16 if cdt == "bf16" else torch().float32, device="cuda")
    from sejong_amd import _native as N_
    wsb = ws(N_.load().sj_gemm_workspace_bytes(M, N, K))
    api.sj_gemm(None, ta, tb, M, N, K, p(dA), DT[adt], A.shape[1], p(dB), DT[bdt], B.shape[1], p(C), DT[cdt], N, 0,
                p(wsb), wsb.numel())
    sync()
    got = host(C)
    if cdt == "bf16":
        assert_stored_close(got, ref, "bf16", "gemm")
    else:
        tol = 1e-5 if (adt == "bf16" and bdt == "bf16") else 6e-5
        assert rel(got, ref) < tol, rel(got, ref)


def test_gemm_accumulate(api):
    rng = np.random.default_rng(7)
    M, N, K = 384, 384, 4096
    A = rnd((K, M), "bf16", rng); B = rng.normal(0, 1, (K, N)).astype(np.float32).astype(np.float64)
    C0 = rng.normal(0, 1, (M, N)).astype(np.float32).astype(np.float64)
    C = dev(C0)
    from sejong_amd import _native as N_
    wsb = ws(N_.load().sj_gemm_workspace_bytes(M, N, K))
    api.sj_gemm(None, 1, 0, M, N, K, p(dev(A, "bf16")), BF, M, p(dev(B)), F32, N, p(C), F32, N, 1, p(wsb), wsb.numel())
    sync()
    assert rel(host(C), C0 + O.matmul(A, B, 1, 0)) < 6e-5


# --------------------------------------------------- fused projections
def rope_table(T, Dh, theta=10000.0):
    t = torch().empty(T * Dh, device="cuda")
    from sejong_amd import _native as N
    N.api.sj_rope_table(None, p(t), T, Dh, ctypes.c_float(theta))
    return t


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_qkv_rope_fused(api, dt):
    rng = np.random.default_rng(3)
    T, B, D, HQ, HK = 128, 2, 128, 2, 1
    Dh = D // HQ; J = HK * Dh; M = T * B
    x = rnd((M, D), dt, rng); wq = rnd((D, D), dt, rng, 0.1); wk = rnd((D, J), dt, rng, 0.1); wv = rnd((D, J), dt, rng, 0.1)
    NQ = D + 2 * J
    out = torch().empty((M, NQ), dtype=torch().bfloat16 if dt == "bf16" else torch().float32, device="cuda")
    es = 2 if dt == "bf16" else 4
    tab = rope_table(T, Dh)
    base = out.data_ptr()
    api.sj_qkv_fwd(None, p(dev(x, dt)), D, M, D, p(dev(wq, dt)), D, p(dev(wk, dt)), J, p(dev(wv, dt)), J, D, J,
                   ctypes.c_void_p(base), NQ, ctypes.c_void_p(base + D * es), NQ, ctypes.c_void_p(base + (D + J) * es), NQ,
                   DT[dt], p(tab), T, Dh)
    sync()
    got = host(out)
    q = O.round_to(x @ wq, dt); k = O.round_to(x @ wk, dt); v = O.matmul(x, wv)
    assert_stored_close(got[:, :D], O.rope(q, T, HQ, Dh), dt, "q")
    assert_stored_close(got[:, D:D + J], O.rope(k, T, HK, Dh), dt, "k")
    assert_stored_close(got[:, D + J:], v, dt, "v")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_gate_up_and_residual(api, dt):
    rng = np.random.default_rng(4)
    M, D, F = 512, 128, 384
    x = rnd((M, D), dt, rng); wg = rnd((D, F), dt, rng, 0.1); wu = rnd((D, F), dt, rng, 0.1)
    wgu = np.concatenate([wg, wu], 1)
    tt = torch().bfloat16 if dt == "bf16" else torch().float32
    G, U, H = (torch().empty((M, F), dtype=tt, device="cuda") for _ in range(3))
    W = dev(wgu, dt)
    es = 2 if dt == "bf16" else 4
    api.sj_gate_up_fwd(None, p(dev(x, dt)), D, M, D, p(W), 2 * F, ctypes.c_void_p(W.data_ptr() + F * es), 2 * F, F,
                       p(G), p(U), p(H), F, DT[dt])
    sync()
    g = O.round_to(x @ wg, dt); u = O.round_to(x @ wu, dt)
    assert_stored_close(host(G), O.matmul(x, wg), dt, "g")
    assert_stored_close(host(U), O.matmul(x, wu), dt, "u")
    assert_stored_close(host(H), O.swiglu_fwd(g, u), dt, "h")
    # residual projection: y = r + round(h Wd)
    h = O.round_to(O.swiglu_fwd(g, u), dt)
    wd = rnd((F, D), dt, rng, 0.1); r = rnd((M, D), dt, rng)
    Y = torch().empty((M, D), dtype=tt, device="cuda")
    api.sj_linear_residual_fwd(None, p(dev(h, dt)), F, M, F, p(dev(wd, dt)), D, D, p(dev(r, dt)), D, p(Y), D, DT[dt])
    sync()
    assert_stored_close(host(Y), r + O.round_to(h @ wd, dt), dt, "residual")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_down_backward_swiglu(api, dt):
    rng = np.random.default_rng(5)
    M, D, F = 512, 128, 384
    dy = rng.normal(0, 1e-4, (M, D)).astype(np.float32).astype(np.float64)
    wd = rnd((F, D), dt, rng, 0.1); g = rnd((M, F), dt, rng); u = rnd((M, F), dt, rng)
    dgu = torch().empty((M, 2 * F), device="cuda")
    api.sj_down_bwd_swiglu(None, p(dev(dy)), D, M, D, p(dev(wd, dt)), D, F, p(dev(g, dt)), p(dev(u, dt)), F, DT[dt],
                           p(dgu), 2 * F)
    sync()
    dh = O.matmul(dy, wd, 0, 1)
    dg, du = O.swiglu_bwd(g, u, dh)
    got = host(dgu)
    assert rel(got[:, :F], dg) < 6e-5 and rel(got[:, F:], du) < 6e-5


# ----------------------------------------------------------- attention
ATT_CASES = [
    # B, T, HQ, HK, Dh, dt, window
    (2, 256, 6, 2, 64, "bf16", 0),   # MFMA path
    (1, 200, 4, 4, 64, "bf16", 0),   # MFMA path, ragged T, MHA
    (2, 128, 4, 2, 32, "f32", 0),    # row kernels (cfg1 shape)
    (1, 96, 4, 2, 64, "bf16", 24),   # row kernels, sliding window
]


@pytest.mark.parametrize("B,T,HQ,HK,Dh,dt,window", ATT_CASES)
def test_attention(api, B, T, HQ, HK, Dh, dt, window):
    rng = np.random.default_rng(B * T + HQ)
    M = B * T
    q = rnd((M, HQ * Dh), dt, rng); k = rnd((M, HK * Dh), dt, rng); v = rnd((M, HK * Dh), dt, rng)
    do = rng.normal(0, 1e-4, (M, HQ * Dh)).astype(np.float32).astype(np.float64)
    tt = torch().bfloat16 if dt == "bf16" else torch().float32
    Q, K, V, DO = dev(q, dt), dev(k, dt), dev(v, dt), dev(do)
    Ot = torch().empty((M, HQ * Dh), dtype=tt, device="cuda"); L = torch().empty(M * HQ, device="cuda")
    api.sj_attention_fwd(None, p(Q), HQ * Dh, p(K), HK * Dh, p(V), HK * Dh, p(Ot), HQ * Dh, p(L), DT[dt], B, T, HQ, HK, Dh, window)
    sync()
    o_ref, lse_ref = O.attention_fwd(q, k, v, B, T, HQ, HK, Dh, window)
    assert_stored_close(host(Ot), o_ref, dt, "O")
    assert rel(host(L), lse_ref) < 1e-6
    # backward conditioned on the stored O and LSE (as the reference does)
    o_st, lse_st = host(Ot), host(L)
    dQ = torch().empty((M, HQ * Dh), device="cuda"); dK = torch().empty((M, HK * Dh), device="cuda")
    dV = torch().empty((M, HK * Dh), device="cuda"); De = torch().empty(M * HQ, device="cuda")
    for use_rope in (False, True):
        tab = rope_table(T, Dh) if use_rope else None
        api.sj_attention_bwd(None, p(Q), HQ * Dh, p(K), HK * Dh, p(V), HK * Dh, p(Ot), HQ * Dh, p(L), p(DO), HQ * Dh,
                             p(dQ), HQ * Dh, p(dK), HK * Dh, p(dV), HK * Dh, p(De), DT[dt], B, T, HQ, HK, Dh, window,
                             p(tab) if tab is not None else None)
        sync()
        dq, dk, dv, delta = O.attention_bwd(q, k, v, o_st, lse_st, do, B, T, HQ, HK, Dh, window)
        if use_rope:
            dq = O.rope(dq, T, HQ, Dh, inverse=True); dk = O.rope(dk, T, HK, Dh, inverse=True)
        assert rel(host(De), delta) < 1e-5
        for name, got, ref in (("dq", dQ, dq), ("dk", dK, dk), ("dv", dV, dv)):
            r = rel(host(got), ref)
            assert r < 1e-4, (name, use_rope, r)


# -------------------------------------------------- CE, embedding, misc
def test_cross_entropy_and_loss_summary(api):
    rng = np.random.default_rng(6)
    R, V, Vp = 1000, 257, 264
    x = rng.normal(0, 2, (R, Vp)).astype(np.float32).astype(np.float64)
    t = rng.integers(0, 256, R).astype(np.int32)
    X = dev(x); L = torch().empty(R, device="cuda"); DX = torch().zeros((R, Vp), device="cuda")
    api.sj_cross_entropy(None, p(X), Vp, p(dev(t, "i32")), p(L), p(DX), Vp, R, V, None, ctypes.c_float(1.0 / R))
    out = torch().zeros(4, dtype=torch().float64, device="cuda")
    api.sj_loss_summary(None, p(L), R, p(out), 1, ctypes.c_float(0.5))
    sync()
    loss, dx = O.cross_entropy(x[:, :V], t, float(np.float32(1.0 / R)))
    assert rel(host(L), loss) < 1e-6 and rel(host(DX)[:, :V], dx) < 1e-6
    assert np.all(host(DX)[:, V:] == 0)
    assert abs(out[1].item() - host(L).sum() * 0.5 / R) < 1e-9 * abs(out[1].item())


def test_embedding_forward_backward(api):
    rng = np.random.default_rng(8)
    V, D, Nn = 257, 384, 3000
    W = rnd((V, D), "bf16", rng); ids = rng.integers(0, 256, Nn).astype(np.int32); ids[:5] = 256
    Y = torch().empty((Nn, D), dtype=torch().bfloat16, device="cuda")
    I = dev(ids, "i32")
    api.sj_embedding_fwd(None, p(dev(W, "bf16")), BF, p(I), p(Y), BF, Nn, D)
    dy = rng.normal(0, 1, (Nn, D)).astype(np.float32).astype(np.float64)
    dW = torch().full((V, D), 7.0, device="cuda")
    api.sj_embedding_bwd(None, p(dev(dy)), p(I), p(dW), Nn, D, V, None, 0)
    sync()
    np.testing.assert_array_equal(host(Y), W[ids])
    assert rel(host(dW), O.embedding_bwd(dy, ids, V)) < 1e-6


def test_sum_squares_and_adamw(api):
    rng = np.random.default_rng(9)
    n = 1_000_003
    g = rng.normal(0, 1e-3, n).astype(np.float32).astype(np.float64)
    G = dev(g); out = torch().zeros(1, dtype=torch().float64, device="cuda")
    from sejong_amd import _native as N
    wsb = ws(N.load().sj_sum_squares_workspace_bytes(n))
    api.sj_sum_squares(None, p(G), n, p(out), p(wsb), wsb.numel())
    sync()
    assert abs(out.item() - O.sum_squares(g)) < 1e-12 * O.sum_squares(g)
    w = rng.normal(0, 0.02, n).astype(np.float32).astype(np.float64)
    m = rng.normal(0, 1e-4, n).astype(np.float32).astype(np.float64)
    v = np.abs(rng.normal(0, 1e-7, n)).astype(np.float32).astype(np.float64)
    W, M_, V_ = dev(w), dev(m), dev(v)
    args = dict(lr=3e-4, b1=0.9, b2=0.95, eps=0.0, decay=0.01, ib1=1 / (1 - 0.9 ** 3), ib2=1 / (1 - 0.95 ** 3), scale=0.7)
    f = [ctypes.c_float(args[k]) for k in ("lr", "b1", "b2", "eps", "decay", "ib1", "ib2", "scale")]
    api.sj_adamw(None, p(W), p(G), p(M_), p(V_), n, *f)
    sync()
    wr, mr, vr = O.adamw(w, g, m, v, *[float(np.float32(args[k])) for k in ("lr", "b1", "b2", "eps", "decay", "ib1", "ib2", "scale")])
    assert np.max(np.abs(host(W) - wr)) < 2e-7 and rel(host(M_), mr) < 1e-6 and rel(host(V_), vr) < 1e-6


def test_adamw_multi_clip_and_mirror(api):
    from sejong_amd import _native as N
    rng = np.random.default_rng(10)
    n, nd = 10_001, 1_000
    g = rng.normal(0, 1.0, n).astype(np.float32).astype(np.float64)  # norm ~ 100 > clip 1
    w = rng.normal(0, 0.02, n).astype(np.float32).astype(np.float64)
    W, G = dev(w), dev(g)
    M_ = torch().zeros(n, device="cuda"); V_ = torch().zeros(n, device="cuda")
    mir = torch().zeros(n, dtype=torch().bfloat16, device="cuda")
    ss = torch().tensor([O.sum_squares(g)], dtype=torch().float64, device="cuda")
    st = N.AdamStep(lr=1e-3, beta1=0.9, beta2=0.95, eps=0.0, weight_decay=0.1, inv_b1=1 / (1 - np.float32(0.9)),
                    inv_b2=1 / (1 - np.float32(0.95)), clip_norm=1.0, loss_scale=1.0, clip_enabled=1)
    stb = torch().tensor(np.frombuffer(bytes(st), dtype=np.uint8).copy(), device="cuda")
    flag = torch().zeros(1, dtype=torch().int32, device="cuda")
    api.sj_adamw_multi(None, p(W), p(G), p(M_), p(V_), p(mir), n, nd, p(stb), p(ss), p(flag))
    sync()
    norm = math.sqrt(O.sum_squares(g))
    scale = float(np.float32(1.0 / norm))
    wr = np.concatenate([O.adamw(w[:nd], g[:nd], np.zeros(nd), np.zeros(nd), 1e-3, 0.9, 0.95, 0, 0.0, st.inv_b1, st.inv_b2, scale)[0],
                         O.adamw(w[nd:], g[nd:], np.zeros(n - nd), np.zeros(n - nd), 1e-3, 0.9, 0.95, 0, 0.1, st.inv_b1, st.inv_b2, scale)[0]])
    assert np.max(np.abs(host(W) - wr)) < 2e-7
    np.testing.assert_array_equal(host(mir), O.round_to(host(W), "bf16"))
    assert flag.item() == 0
    # non-finite norm: flag set, nothing updated
    ss.fill_(float("inf"))
    before = host(W)
    api.sj_adamw_multi(None, p(W), p(G), p(M_), p(V_), p(mir), n, nd, p(stb), p(ss), p(flag))
    sync()
    assert flag.item() == 1 and np.array_equal(host(W), before)
