"""Per-op parity of the HIP kernels against the FP64 oracle on identical
(storage-rounded) inputs.  Every call goes through the C ABI."""
import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import Dev, assert_stored_close, dev, empty, rel, rnd, sync, zeros

pytestmark = pytest.mark.gpu

BF, F32 = 4, 0
DT = {"bf16": BF, "f32": F32}
cf = ctypes.c_float


@pytest.fixture(scope="module")
def api():
    from sejong_amd import _native as N
    N.load()
    return N.api


@pytest.fixture(scope="module")
def lib():
    from sejong_amd import _native as N
    return N.load()


def ws(nbytes):
    return empty(max(int(nbytes), 256), "u8")


# ------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("dt,R,D", [("bf16", 1000, 384), ("f32", 256, 128), ("bf16", 33, 1024)])
def test_rmsnorm_forward_backward(api, lib, dt, R, D):
    rng = np.random.default_rng(1)
    x = rnd((R, D), dt, rng); w = rnd(D, dt, rng)
    dy = rng.normal(0, 1e-3, (R, D)).astype(np.float32).astype(np.float64)
    acc = rng.normal(0, 1e-3, (R, D)).astype(np.float32).astype(np.float64)
    eps = 1e-6
    X, W, DY, ACC = dev(x, dt), dev(w, dt), dev(dy), dev(acc)
    Y = empty(R * D, dt)
    api.sj_rmsnorm_fwd(None, X.p, DT[dt], W.p, DT[dt], Y.p, R, D, cf(eps))
    DX, DWt = empty(R * D), empty(D)
    wsb = ws(lib.sj_rmsnorm_bwd_workspace_bytes(R, D))
    api.sj_rmsnorm_bwd(None, X.p, DT[dt], W.p, DT[dt], DY.p, ACC.p, DX.p, DWt.p, R, D, cf(eps), wsb.p, wsb.nbytes)
    sync()
    assert_stored_close(Y.host(), O.rmsnorm_fwd(x, w, eps), dt, "rmsnorm y")
    dx, dw = O.rmsnorm_bwd(x, w, dy, eps, dx_acc=acc)
    assert rel(DX.host(), dx) < 1e-5 and rel(DWt.host(), dw) < 1e-5


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
def test_gemm(api, lib, M, N, K, ta, tb, adt, bdt, cdt):
    rng = np.random.default_rng(M + N + K)
    A = rnd((K, M) if ta else (M, K), adt, rng)
    B = rnd((N, K) if tb else (K, N), bdt, rng)
    ref = O.matmul(A, B, ta, tb)
    dA, dB = dev(A, adt), dev(B, bdt)
    C = zeros(M * N, cdt)
    wsb = ws(lib.sj_gemm_workspace_bytes(M, N, K))
    api.sj_gemm(None, ta, tb, M, N, K, dA.p, DT[adt], A.shape[1], dB.p, DT[bdt], B.shape[1], C.p, DT[cdt], N, 0,
                wsb.p, wsb.nbytes)
    sync()
    got = C.host()
    if cdt == "bf16":
        assert_stored_close(got, ref, "bf16", "gemm", terms=O.matmul(np.abs(A), np.abs(B), ta, tb))
    else:
        tol = 1e-5 if (adt == "bf16" and bdt == "bf16") else 6e-5
        assert rel(got, ref) < tol, rel(got, ref)


def test_gemm_accumulate(api, lib):
    rng = np.random.default_rng(7)
    M, N, K = 384, 384, 4096
    A = rnd((K, M), "bf16", rng); B = rng.normal(0, 1, (K, N)).astype(np.float32).astype(np.float64)
    C0 = rng.normal(0, 1, (M, N)).astype(np.float32).astype(np.float64)
    C = dev(C0)
    wsb = ws(lib.sj_gemm_workspace_bytes(M, N, K))
    api.sj_gemm(None, 1, 0, M, N, K, dev(A, "bf16").p, BF, M, dev(B).p, F32, N, C.p, F32, N, 1, wsb.p, wsb.nbytes)
    sync()
    assert rel(C.host(), C0.ravel() + O.matmul(A, B, 1, 0).ravel()) < 6e-5


# --------------------------------------------------- fused projections
def rope_table(api, T, Dh, theta=10000.0):
    t = empty(T * Dh)
    api.sj_rope_table(None, t.p, T, Dh, cf(theta))
    return t


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_qkv_rope_fused(api, dt):
    rng = np.random.default_rng(3)
    T, B, D, HQ, HK = 128, 2, 128, 2, 1
    Dh = D // HQ; J = HK * Dh; M = T * B
    x = rnd((M, D), dt, rng); wq = rnd((D, D), dt, rng, 0.1); wk = rnd((D, J), dt, rng, 0.1); wv = rnd((D, J), dt, rng, 0.1)
    NQ = D + 2 * J
    out = empty(M * NQ, dt)
    tab = rope_table(api, T, Dh)
    api.sj_qkv_fwd(None, dev(x, dt).p, D, M, D, dev(wq, dt).p, D, dev(wk, dt).p, J, dev(wv, dt).p, J, D, J,
                   out.p, NQ, out.at(D), NQ, out.at(D + J), NQ, DT[dt], tab.p, T, Dh)
    sync()
    got = out.host().reshape(M, NQ)
    q = O.round_to(x @ wq, dt); k = O.round_to(x @ wk, dt)
    # RoPE of a rounded value, stored again: each output mixes a pair, so the
    # bound is one ulp of the pair's magnitude for each of the two roundings
    def pairmax(a, H):
        return np.repeat(np.abs(a).reshape(M, H, Dh // 2, 2).max(-1), 2, -1).reshape(M, H * Dh)
    aq = O.matmul(np.abs(x), np.abs(wq)); ak = O.matmul(np.abs(x), np.abs(wk))
    assert_stored_close(got[:, :D], O.rope(q, T, HQ, Dh), dt, "q", ulps=2, terms=pairmax(aq, HQ) + 2 ** 10 * pairmax(q, HQ))
    assert_stored_close(got[:, D:D + J], O.rope(k, T, HK, Dh), dt, "k", ulps=2, terms=pairmax(ak, HK) + 2 ** 10 * pairmax(k, HK))
    assert_stored_close(got[:, D + J:], O.matmul(x, wv), dt, "v", terms=O.matmul(np.abs(x), np.abs(wv)))


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_gate_up_and_residual(api, dt):
    rng = np.random.default_rng(4)
    M, D, F = 512, 128, 384
    x = rnd((M, D), dt, rng); wg = rnd((D, F), dt, rng, 0.1); wu = rnd((D, F), dt, rng, 0.1)
    W = dev(np.concatenate([wg, wu], 1), dt)
    G, U, H = empty(M * F, dt), empty(M * F, dt), empty(M * F, dt)
    api.sj_gate_up_fwd(None, dev(x, dt).p, D, M, D, W.p, 2 * F, W.at(F), 2 * F, F, G.p, U.p, H.p, F, DT[dt])
    sync()
    assert_stored_close(G.host(), O.matmul(x, wg), dt, "g", terms=O.matmul(np.abs(x), np.abs(wg)))
    assert_stored_close(U.host(), O.matmul(x, wu), dt, "u", terms=O.matmul(np.abs(x), np.abs(wu)))
    g, u = G.host().reshape(M, F), U.host().reshape(M, F)  # h is formed from the stored g, u
    assert_stored_close(H.host(), O.swiglu_fwd(g, u), dt, "h")
    h = H.host().reshape(M, F)
    wd = rnd((F, D), dt, rng, 0.1); r = rnd((M, D), dt, rng)
    Y = empty(M * D, dt)
    api.sj_linear_residual_fwd(None, dev(h, dt).p, F, M, F, dev(wd, dt).p, D, D, dev(r, dt).p, D, Y.p, D, DT[dt])
    sync()
    # y = round(r + round(h Wd)): one ulp of each rounding, measured on the
    # larger of the matmul term and the result
    a = O.matmul(h, wd)
    assert_stored_close(Y.host(), r + a, dt, "residual", ulps=2,
                        terms=O.matmul(np.abs(h), np.abs(wd)) + 2 ** 9 * np.abs(a))


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_down_backward_swiglu(api, dt):
    rng = np.random.default_rng(5)
    M, D, F = 512, 128, 384
    dy = rng.normal(0, 1e-4, (M, D)).astype(np.float32).astype(np.float64)
    wd = rnd((F, D), dt, rng, 0.1); g = rnd((M, F), dt, rng); u = rnd((M, F), dt, rng)
    dgu = empty(M * 2 * F)
    api.sj_down_bwd_swiglu(None, dev(dy).p, D, M, D, dev(wd, dt).p, D, F, dev(g, dt).p, dev(u, dt).p, F, DT[dt],
                           dgu.p, 2 * F)
    sync()
    dg, du = O.swiglu_bwd(g, u, O.matmul(dy, wd, 0, 1))
    got = dgu.host().reshape(M, 2 * F)
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
    Q, K, V, DO = dev(q, dt), dev(k, dt), dev(v, dt), dev(do)
    Ot, L = empty(M * HQ * Dh, dt), empty(M * HQ)
    print(f"[attention] B={B} T={T} HQ={HQ} HK={HK} Dh={Dh} {dt} window={window}", flush=True)
    api.sj_attention_fwd(None, Q.p, HQ * Dh, K.p, HK * Dh, V.p, HK * Dh, Ot.p, HQ * Dh, L.p, DT[dt], B, T, HQ, HK, Dh, window)
    sync()
    o_ref, lse_ref = O.attention_fwd(q, k, v, B, T, HQ, HK, Dh, window)
    o_abs, _ = O.attention_fwd(q, k, np.abs(v), B, T, HQ, HK, Dh, window)  # sum_j p_j |v_j|
    assert_stored_close(Ot.host(), o_ref, dt, "O", terms=2 * o_abs)
    assert rel(L.host(), lse_ref) < 1e-5
    # backward conditioned on the stored O and LSE (as the reference does)
    o_st, lse_st = Ot.host().reshape(M, HQ * Dh), L.host()
    dQ, dK, dV, De = empty(M * HQ * Dh), empty(M * HK * Dh), empty(M * HK * Dh), empty(M * HQ)
    for use_rope in (False, True):
        tab = rope_table(api, T, Dh) if use_rope else None
        api.sj_attention_bwd(None, Q.p, HQ * Dh, K.p, HK * Dh, V.p, HK * Dh, Ot.p, HQ * Dh, L.p, DO.p, HQ * Dh,
                             dQ.p, HQ * Dh, dK.p, HK * Dh, dV.p, HK * Dh, De.p, DT[dt], B, T, HQ, HK, Dh, window,
                             tab.p if tab is not None else None)
        sync()
        dq, dk, dv, delta = O.attention_bwd(q, k, v, o_st, lse_st, do, B, T, HQ, HK, Dh, window)
        if use_rope:
            dq = O.rope(dq, T, HQ, Dh, inverse=True); dk = O.rope(dk, T, HK, Dh, inverse=True)
        assert rel(De.host(), delta) < 1e-5
        for name, got, ref in (("dq", dQ, dq), ("dk", dK, dk), ("dv", dV, dv)):
            r = rel(got.host(), ref)
            assert r < 1e-4, (name, use_rope, r)


# -------------------------------------------------- CE, embedding, misc
def test_cross_entropy_and_loss_summary(api):
    rng = np.random.default_rng(6)
    R, V, Vp = 1000, 257, 264
    x = rng.normal(0, 2, (R, Vp)).astype(np.float32).astype(np.float64)
    t = rng.integers(0, 256, R).astype(np.int32)
    X = dev(x); L = empty(R); DX = zeros(R * Vp)
    api.sj_cross_entropy(None, X.p, Vp, dev(t, "i32").p, L.p, DX.p, Vp, R, V, None, cf(1.0 / R))
    out = zeros(4, "f64")
    api.sj_loss_summary(None, L.p, R, out.p, 1, cf(0.5))
    sync()
    loss, dx = O.cross_entropy(x[:, :V], t, float(np.float32(1.0 / R)))
    got_dx = DX.host().reshape(R, Vp)
    assert rel(L.host(), loss) < 1e-6 and rel(got_dx[:, :V], dx) < 1e-6
    assert np.all(got_dx[:, V:] == 0)
    s = out.host()[1]
    assert abs(s - L.host().sum() * 0.5 / R) < 1e-9 * abs(s)


def _bf16_rne(x32):
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.asarray(x32, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("xd,yd", [("f32", "f32"), ("bf16", "bf16"), ("f32", "bf16"), ("bf16", "f32")])
def test_cast_copy_bits_offsets_and_tails(api, xd, yd):
    """Engine::cast / copy_into (kernels.py:11-14): the same-dtype copy moves
    the bits (NaN payloads, signed zeros, denormals included), through the
    16-byte vector path when both pointers are aligned and the element loop
    for the rest; f32 -> bf16 rounds to nearest even; nothing outside
    y[0, n) is written."""
    rng = np.random.default_rng(8)
    item = {"f32": 4, "bf16": 2}
    for n in (1, 3, 4, 5, 8, 9, 1000, 4099, 300001):
        for xo, yo in ((0, 0), (item[xd], 0), (0, item[yd]), (16, 16)):
            if xd == "f32" and yd == "f32":  # any bits: a NaN payload, -0, the smallest denormal
                xbits = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
                xbits[:3] = np.array([0x7FC01234, 0x80000000, 0x00000001], np.uint32)[:min(n, 3)]
            elif xd == "f32":  # finite values for the rounding check
                xbits = rng.normal(0, 3, n).astype(np.float32).view(np.uint32)
            else:
                xbits = _bf16_rne(rng.normal(0, 3, n).astype(np.float32))
                if yd == "bf16":
                    xbits[:2] = np.array([0x7FC1, 0x8000], np.uint16)[:min(n, 2)]
            xraw = xbits.view(np.uint8)
            X = dev(np.concatenate([np.zeros(xo, np.uint8), xraw]), "u8")
            guard = np.full(yo + n * item[yd] + 64, 0xA5, np.uint8)
            Y = dev(guard, "u8")
            print(f"[cast] {xd}->{yd} n {n} offsets {xo}/{yo}", flush=True)
            api.sj_cast(None, ctypes.c_void_p(X.ptr + xo), DT[xd], ctypes.c_void_p(Y.ptr + yo), DT[yd], n)
            sync()
            got = Y.host()
            assert np.all(got[:yo] == 0xA5) and np.all(got[yo + n * item[yd]:] == 0xA5), (n, xo, yo)
            body = got[yo:yo + n * item[yd]]
            if xd == yd:
                want = xraw
            elif yd == "bf16":
                want = _bf16_rne(xbits.view(np.float32)).view(np.uint8)
            else:
                want = (xbits.astype(np.uint32) << 16).view(np.uint8)
            np.testing.assert_array_equal(body, want, err_msg=f"{xd}->{yd} n {n} offsets {xo}/{yo}")


def test_embedding_forward_backward(api):
    rng = np.random.default_rng(8)
    V, D, Nn = 257, 384, 3000
    W = rnd((V, D), "bf16", rng); ids = rng.integers(0, 256, Nn).astype(np.int32); ids[:5] = 256
    Y = empty(Nn * D, "bf16")
    I = dev(ids, "i32")
    api.sj_embedding_fwd(None, dev(W, "bf16").p, BF, I.p, Y.p, BF, Nn, D)
    dy = rng.normal(0, 1, (Nn, D)).astype(np.float32).astype(np.float64)
    dW = dev(np.full(V * D, 7.0))
    api.sj_embedding_bwd(None, dev(dy).p, I.p, dW.p, Nn, D, V, None, 0)
    sync()
    np.testing.assert_array_equal(Y.host().reshape(Nn, D), W[ids])
    assert rel(dW.host(), O.embedding_bwd(dy, ids, V)) < 1e-6


@pytest.mark.parametrize("V,D,Nn,same", [(257, 384, 9000, False), (257, 64, 5000, True), (259, 130, 700, False),
                                         (257, 1024, 4096, False)])
def test_embedding_backward_token_order(api, V, D, Nn, same):
    """The embedding backward sums each row's tokens in token order in fp32
    (deterministic; bit-equal to that sequential sum): several 4096-token
    scan rounds, every token on one id (4096 matches in a round), a width
    that is not a multiple of 4 (the per-column kernel)."""
    rng = np.random.default_rng(V + D + Nn)
    ids = (np.full(Nn, 7) if same else rng.integers(0, V, Nn)).astype(np.int32)
    dy = rng.normal(0, 1, (Nn, D)).astype(np.float32)
    dW = dev(np.full(V * D, 7.0))
    print(f"[embedding_bwd] V={V} D={D} N={Nn} same={same}", flush=True)
    api.sj_embedding_bwd(None, dev(dy.astype(np.float64)).p, dev(ids, "i32").p, dW.p, Nn, D, V, None, 0)
    sync()
    ref = np.zeros((V, D), np.float32)
    for i in range(Nn):
        ref[ids[i]] += dy[i]
    np.testing.assert_array_equal(dW.host().reshape(V, D).astype(np.float32), ref)


def test_sum_squares_and_adamw(api, lib):
    rng = np.random.default_rng(9)
    n = 1_000_003
    g = rng.normal(0, 1e-3, n).astype(np.float32).astype(np.float64)
    G = dev(g); out = zeros(1, "f64")
    wsb = ws(lib.sj_sum_squares_workspace_bytes(n))
    api.sj_sum_squares(None, G.p, n, out.p, wsb.p, wsb.nbytes)
    sync()
    assert abs(out.host()[0] - O.sum_squares(g)) < 1e-12 * O.sum_squares(g)
    w = rng.normal(0, 0.02, n).astype(np.float32).astype(np.float64)
    m = rng.normal(0, 1e-4, n).astype(np.float32).astype(np.float64)
    v = np.abs(rng.normal(0, 1e-7, n)).astype(np.float32).astype(np.float64)
    W, M_, V_ = dev(w), dev(m), dev(v)
    args = [3e-4, 0.9, 0.95, 0.0, 0.01, 1 / (1 - 0.9 ** 3), 1 / (1 - 0.95 ** 3), 0.7]
    api.sj_adamw(None, W.p, G.p, M_.p, V_.p, n, *[cf(a) for a in args])
    sync()
    wr, mr, vr = O.adamw(w, g, m, v, *[float(np.float32(a)) for a in args])
    assert np.max(np.abs(W.host() - wr)) < 2e-7 and rel(M_.host(), mr) < 1e-6 and rel(V_.host(), vr) < 1e-6


def test_adamw_multi_clip_and_mirror(api):
    from sejong_amd import _native as N
    rng = np.random.default_rng(10)
    n, nd = 10_001, 1_000
    g = rng.normal(0, 1.0, n).astype(np.float32).astype(np.float64)  # norm ~ 100 > clip 1
    w = rng.normal(0, 0.02, n).astype(np.float32).astype(np.float64)
    W, G = dev(w), dev(g)
    M_, V_, mir = zeros(n), zeros(n), zeros(n, "bf16")
    ss = dev(np.array([O.sum_squares(g)]), "f64")
    st = N.AdamStep(lr=1e-3, beta1=0.9, beta2=0.95, eps=0.0, weight_decay=0.1, inv_b1=1 / (1 - np.float32(0.9)),
                    inv_b2=1 / (1 - np.float32(0.95)), clip_norm=1.0, loss_scale=1.0, clip_enabled=1)
    stb = dev(np.frombuffer(bytes(st), dtype=np.uint8), "u8")
    flag = zeros(1, "i32")
    api.sj_adamw_multi(None, W.p, G.p, M_.p, V_.p, mir.p, n, nd, stb.p, ss.p, flag.p)
    sync()
    scale = float(np.float32(1.0 / math.sqrt(O.sum_squares(g))))
    wr = np.concatenate([
        O.adamw(w[:nd], g[:nd], np.zeros(nd), np.zeros(nd), 1e-3, 0.9, 0.95, 0, 0.0, st.inv_b1, st.inv_b2, scale)[0],
        O.adamw(w[nd:], g[nd:], np.zeros(n - nd), np.zeros(n - nd), 1e-3, 0.9, 0.95, 0, 0.1, st.inv_b1, st.inv_b2, scale)[0]])
    got = W.host()
    assert np.max(np.abs(got - wr)) < 2e-7
    np.testing.assert_array_equal(mir.host(), O.round_to(got, "bf16"))
    assert flag.host()[0] == 0
    # non-finite norm: flag set, nothing updated
    ss.upload(np.array([np.inf]))
    api.sj_adamw_multi(None, W.p, G.p, M_.p, V_.p, mir.p, n, nd, stb.p, ss.p, flag.p)
    sync()
    assert flag.host()[0] == 1 and np.array_equal(W.host(), got)
