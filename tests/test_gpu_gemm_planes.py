"""Parity of the MFMA-layout GEMM family (bf16 k-contiguous planes, LDS-DMA
streaming) against the FP64 oracle."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import assert_stored_close, dev, empty, rel, rnd, sync, zeros

pytestmark = pytest.mark.gpu

BF, F32 = 4, 0
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


def split(x):
    """fp32 value -> (hi, lo) bf16 planes as float64 arrays."""
    x32 = np.asarray(x, np.float32).astype(np.float64)
    hi = O.round_to(x32, "bf16")
    return hi, O.round_to(x32 - hi, "bf16")


PLANE_CASES = [
    # M, N, K, split_a, split_b, cdt
    (4096, 640, 384, False, False, "f32"),
    (4096, 384, 2048, True, False, "f32"),      # dX with split dY
    (384, 640, 4096, False, True, "f32"),       # dW with split dY^T, split-K
    (1000, 200, 200, False, False, "bf16"),     # edges: ragged M/N, K % 64 != 0
    (384, 384, 4096, True, False, "f32"),
    (130, 1030, 72, False, True, "f32"),
    # token-split k-contiguous kernel (B one plane, K a multiple of 128):
    # ragged M and N, bf16 output, split K, odd step counts
    (1000, 264, 384, False, False, "bf16"),
    (136, 100, 1280, True, False, "f32"),
    (4096, 384, 640, True, False, "f32"),
]


@pytest.mark.parametrize("M,N,K,sa,sb,cdt", PLANE_CASES)
def test_gemm_planes(api, lib, M, N, K, sa, sb, cdt):
    rng = np.random.default_rng(M * 7 + N + K)
    A = rng.normal(0, 1, (M, K)).astype(np.float32).astype(np.float64)
    B = rng.normal(0, 1, (N, K)).astype(np.float32).astype(np.float64)
    if not sa:
        A = O.round_to(A, "bf16")
    if not sb:
        B = O.round_to(B, "bf16")
    ah, al = split(A) if sa else (A, None)
    bh, bl = split(B) if sb else (B, None)
    dAh, dBh = dev(ah, "bf16"), dev(bh, "bf16")
    dAl = dev(al, "bf16") if sa else None
    dBl = dev(bl, "bf16") if sb else None
    C = zeros(M * N, cdt)
    ws = empty(max(lib.sj_gemm_planes_workspace_bytes(M, N, K), 256), "u8")
    api.sj_gemm_planes(None, M, N, K, dAh.p, dAl.p if sa else None, K, dBh.p, dBl.p if sb else None, K, C.p,
                       BF if cdt == "bf16" else F32, N, 0, ws.p, ws.nbytes)
    sync()
    ref = O.matmul(A, B, 0, 1)
    if cdt == "bf16":
        assert_stored_close(C.host(), ref, "bf16", "planes", terms=O.matmul(np.abs(A), np.abs(B), 0, 1))
    else:
        r = rel(C.host(), ref)
        assert r < (1e-5 if not (sa or sb) else 3e-5), r


TN_CASES = [
    # M, N, K (tokens), split_x, split_y: the step's dW shapes and ragged / split-K ones
    (384, 2048, 4096, False, True),    # gate|up dW at cfg2
    (1024, 384, 4096, False, True),    # down dW
    (384, 640, 4096, False, True),     # q|k|v dW
    (136, 200, 1000, False, True),     # M, N not multiples of 64, K not of 64
    (384, 384, 16384, False, True),    # long K: split-K partials
    (256, 192, 512, True, True),       # both operands split
    (64, 64, 40, False, False),        # one tile, K shorter than a stage
    # token-split dW kernel (one X plane, K >= 1024 a multiple of 256):
    # ragged tiles, one or two Y planes, 1..16 K slices
    (136, 200, 1536, False, True),
    (200, 136, 2048, False, False),
    (72, 64, 1280, False, True),
    (64, 1024, 8192, False, True),
    # K >= 1024 not a multiple of 256: the k_gemm_fast form
    (136, 200, 1500, False, True),
    (200, 136, 2056, False, False),
]


@pytest.mark.parametrize("M,N,K,sx,sy", TN_CASES)
def test_gemm_planes_tn_row_layout(api, lib, M, N, K, sx, sy):
    """C = X^T Y from row-layout operands (X [K][M], Y [K][N], fragments by
    LDS transpose reads) against X^T Y in FP64 and sj_gemm_planes on the
    transposed copies (same operand values; the K split may differ)."""
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    X = rng.normal(0, 1, (K, M)).astype(np.float32).astype(np.float64)
    Y = rng.normal(0, 1, (K, N)).astype(np.float32).astype(np.float64)
    if not sx:
        X = O.round_to(X, "bf16")
    if not sy:
        Y = O.round_to(Y, "bf16")
    xh, xl = split(X) if sx else (X, None)
    yh, yl = split(Y) if sy else (Y, None)
    ldx, ldy = M + 8, N + 16                              # padded row strides
    pad = lambda a, ld: np.concatenate([a, np.zeros((a.shape[0], ld - a.shape[1]))], 1)
    Xh, Yh = dev(pad(xh, ldx), "bf16"), dev(pad(yh, ldy), "bf16")
    Xl = dev(pad(xl, ldx), "bf16") if sx else None
    Yl = dev(pad(yl, ldy), "bf16") if sy else None
    ws = empty(max(lib.sj_gemm_planes_workspace_bytes(M, N, K), 256), "u8")
    C = zeros(M * N)
    print(f"[gemm_tn] M={M} N={N} K={K} split x/y {sx}/{sy}", flush=True)
    api.sj_gemm_planes_tn(None, M, N, K, Xh.p, Xl.p if sx else None, ldx, Yh.p, Yl.p if sy else None, ldy, C.p, F32,
                          N, 0, ws.p, ws.nbytes)
    Kp = (K + 7) // 8 * 8                                 # k-contiguous copies need K % 8 == 0
    tr = lambda a: dev(np.concatenate([a.T, np.zeros((a.shape[1], Kp - K))], 1), "bf16")
    C2 = zeros(M * N)
    api.sj_gemm_planes(None, M, N, Kp, tr(xh).p, tr(xl).p if sx else None, Kp, tr(yh).p, tr(yl).p if sy else None,
                       Kp, C2.p, F32, N, 0, ws.p, ws.nbytes)
    sync()
    ref = O.matmul(X, Y, 1, 0)
    assert rel(C.host(), ref) < (1e-5 if not (sx or sy) else 3e-5), rel(C.host(), ref)
    if Kp == K:  # same operand values; the plans may split K differently (fp32 partial sums)
        assert rel(C.host(), C2.host()) < 1e-6


@pytest.mark.parametrize("M,N,K,split_b", [(384, 384, 4096, True), (4096, 384, 2048, False), (256, 384, 4096, False)])
def test_gemm_planes_accumulate(api, lib, M, N, K, split_b):
    """C += A B^T with a split B (k_gemm_fast) or a split A (the token-split
    k-contiguous kernel, unsplit and split-K)."""
    rng = np.random.default_rng(11 + M)
    A = rng.normal(0, 1, (M, K)).astype(np.float32).astype(np.float64)
    B = rng.normal(0, 1, (N, K)).astype(np.float32).astype(np.float64)
    if split_b:
        A = O.round_to(A, "bf16")
        ah, al = A, None
        bh, bl = split(B)
    else:
        B = O.round_to(B, "bf16")
        ah, al = split(A)
        bh, bl = B, None
    C0 = rng.normal(0, 1, (M, N)).astype(np.float32).astype(np.float64)
    C = dev(C0)
    ws = empty(max(lib.sj_gemm_planes_workspace_bytes(M, N, K), 256), "u8")
    api.sj_gemm_planes(None, M, N, K, dev(ah, "bf16").p, dev(al, "bf16").p if al is not None else None, K,
                       dev(bh, "bf16").p, dev(bl, "bf16").p if bl is not None else None, K, C.p, F32, N, 1, ws.p, ws.nbytes)
    sync()
    assert rel(C.host(), (C0 + O.matmul(A, B, 0, 1)).ravel()) < 3e-5


@pytest.mark.parametrize("M,N,K,cdt,accumulate", [(384, 2048, 4096, "f32", 1), (384, 640, 4096, "f32", 1),
                                                  (384, 2048, 4096, "bf16", 0), (384, 640, 4096, "bf16", 0)])
def test_gemm_planes_tn_accumulate_and_bf16(api, lib, M, N, K, cdt, accumulate):
    """Row-layout products with C += X^T Y or a bf16 C, unsplit (the tile
    count fills the CUs) and split-K (partials and their reduce)."""
    rng = np.random.default_rng(M + N + K + accumulate)
    X = O.round_to(rng.normal(0, 1, (K, M)), "bf16")
    Y = rng.normal(0, 1, (K, N)).astype(np.float32).astype(np.float64)
    yh, yl = split(Y)
    C0 = rng.normal(0, 1, (M, N)).astype(np.float32).astype(np.float64) if accumulate else np.zeros((M, N))
    C = dev(C0) if cdt == "f32" else zeros(M * N, "bf16")
    ws = empty(max(lib.sj_gemm_planes_workspace_bytes(M, N, K), 256), "u8")
    print(f"[gemm_tn] M={M} N={N} K={K} {cdt} accumulate {accumulate}", flush=True)
    api.sj_gemm_planes_tn(None, M, N, K, dev(X, "bf16").p, None, M, dev(yh, "bf16").p, dev(yl, "bf16").p, N, C.p,
                          F32 if cdt == "f32" else BF, N, accumulate, ws.p, ws.nbytes)
    sync()
    ref = (C0 + O.matmul(X, Y, 1, 0)).ravel()
    if cdt == "bf16":
        assert_stored_close(C.host(), ref, "bf16", "tn bf16", terms=O.matmul(np.abs(X), np.abs(Y), 1, 0))
    else:
        assert rel(C.host(), ref) < 3e-5


def _pairmax(a, M, H, Dh):
    return np.repeat(np.abs(a).reshape(M, H, Dh // 2, 2).max(-1), 2, -1).reshape(M, H * Dh)


def test_qkv_t_rope(api):
    rng = np.random.default_rng(12)
    T, B, D, HQ, HK = 256, 2, 384, 6, 2
    Dh = D // HQ; J = HK * Dh; M = T * B; NQ = D + 2 * J
    x = O.round_to(rng.normal(0, 1, (M, D)), "bf16")
    w = O.round_to(rng.normal(0, 0.05, (D, NQ)), "bf16")  # [D][q|k|v]
    tab = empty(T * Dh)
    api.sj_rope_table(None, tab.p, T, Dh, cf(10000.0))
    out = empty(M * NQ, "bf16")
    ldt = M + 8
    out_t = zeros(NQ * ldt, "bf16")
    api.sj_qkv_fwd_t(None, dev(x, "bf16").p, D, M, D, dev(w.T.copy(), "bf16").p, D, D, J, out.p, NQ, tab.p, T, Dh,
                     out_t.p, ldt)
    sync()
    got = out.host().reshape(M, NQ)
    # the transposed copy holds the same stored values (q, k after RoPE)
    np.testing.assert_array_equal(out_t.host().reshape(NQ, ldt)[:, :M], got.T)
    q = O.round_to(x @ w[:, :D], "bf16"); k = O.round_to(x @ w[:, D:D + J], "bf16")
    aq = np.abs(x) @ np.abs(w)
    assert_stored_close(got[:, :D], O.rope(q, T, HQ, Dh), "bf16", "q", ulps=2,
                        terms=_pairmax(aq[:, :D], M, HQ, Dh) + 2 ** 10 * _pairmax(q, M, HQ, Dh))
    assert_stored_close(got[:, D:D + J], O.rope(k, T, HK, Dh), "bf16", "k", ulps=2,
                        terms=_pairmax(aq[:, D:D + J], M, HK, Dh) + 2 ** 10 * _pairmax(k, M, HK, Dh))
    assert_stored_close(got[:, D + J:], x @ w[:, D + J:], "bf16", "v", terms=aq[:, D + J:])


def test_gate_up_t_and_residual_t(api):
    rng = np.random.default_rng(13)
    M, D, F = 1024, 384, 1024
    x = O.round_to(rng.normal(0, 1, (M, D)), "bf16")
    wg = O.round_to(rng.normal(0, 0.05, (D, F)), "bf16"); wu = O.round_to(rng.normal(0, 0.05, (D, F)), "bf16")
    G, U, H, HT = (empty(M * F, "bf16") for _ in range(4))
    api.sj_gate_up_fwd_t(None, dev(x, "bf16").p, D, M, D, dev(wg.T.copy(), "bf16").p, dev(wu.T.copy(), "bf16").p, D, F,
                         G.p, U.p, H.p, F, HT.p, M)
    sync()
    ax = np.abs(x)
    assert_stored_close(G.host(), x @ wg, "bf16", "g", terms=ax @ np.abs(wg))
    assert_stored_close(U.host(), x @ wu, "bf16", "u", terms=ax @ np.abs(wu))
    g, u = G.host().reshape(M, F), U.host().reshape(M, F)
    h = H.host().reshape(M, F)
    assert_stored_close(h, O.swiglu_fwd(g, u), "bf16", "h")
    np.testing.assert_array_equal(HT.host().reshape(F, M), h.T)
    wd = O.round_to(rng.normal(0, 0.05, (F, D)), "bf16"); r = O.round_to(rng.normal(0, 1, (M, D)), "bf16")
    Y = empty(M * D, "bf16")
    api.sj_linear_residual_fwd_t(None, H.p, F, M, F, dev(wd.T.copy(), "bf16").p, F, D, dev(r, "bf16").p, D, Y.p, D)
    sync()
    a = h @ wd
    assert_stored_close(Y.host(), r + a, "bf16", "residual", ulps=2,
                        terms=np.abs(h) @ np.abs(wd) + 2 ** 9 * np.abs(a))


@pytest.mark.parametrize("M,F", [(1024, 1024), (1000, 200)])
def test_down_bwd_swiglu_planes(api, M, F):
    rng = np.random.default_rng(14 + M + F)
    D = 384
    dy = rng.normal(0, 1e-4, (M, D)).astype(np.float32).astype(np.float64)
    dh_, dl_ = split(dy)
    wd = O.round_to(rng.normal(0, 0.05, (F, D)), "bf16")
    g = O.round_to(rng.normal(0, 1, (M, F)), "bf16"); u = O.round_to(rng.normal(0, 1, (M, F)), "bf16")
    Hn, Ln, Ht, Lt = (empty(M * 2 * F, "bf16") for _ in range(4))
    api.sj_down_bwd_swiglu_p(None, dev(dh_, "bf16").p, dev(dl_, "bf16").p, D, M, D, dev(wd, "bf16").p, D, F,
                             dev(g, "bf16").p, dev(u, "bf16").p, F, Hn.p, Ln.p, 2 * F, Ht.p, Lt.p, M)
    sync()
    dg, du = O.swiglu_bwd(g, u, O.matmul(dy, wd, 0, 1))
    ref = np.concatenate([dg, du], 1)
    got = (Hn.host() + Ln.host()).reshape(M, 2 * F)
    assert rel(got, ref) < 3e-5
    np.testing.assert_array_equal(Ht.host().reshape(2 * F, M), Hn.host().reshape(M, 2 * F).T)
    np.testing.assert_array_equal(Lt.host().reshape(2 * F, M), Ln.host().reshape(M, 2 * F).T)
    # without transposed outputs the row-plane epilogue (vector G/U prefetch,
    # fp32 dH tile) writes the same planes bit for bit
    Hr, Lr = empty(M * 2 * F, "bf16"), empty(M * 2 * F, "bf16")
    api.sj_down_bwd_swiglu_p(None, dev(dh_, "bf16").p, dev(dl_, "bf16").p, D, M, D, dev(wd, "bf16").p, D, F,
                             dev(g, "bf16").p, dev(u, "bf16").p, F, Hr.p, Lr.p, 2 * F, None, None, M)
    sync()
    np.testing.assert_array_equal(Hr.host(), Hn.host())
    np.testing.assert_array_equal(Lr.host(), Ln.host())
    # hi is the RNE bf16 of the value and lo the rest: |lo| <= half an ulp of hi
    hi, lo = Hn.host(), Ln.host()
    assert np.all(np.abs(lo) <= 2.0 ** -8 * np.abs(hi) + 1e-38)


def _check_planes(hi, lo, x):
    """hi = RNE_bf16(x), lo = RNE_bf16(x - hi), bit for bit (x: the fp32 values)."""
    x = np.asarray(x, np.float32).astype(np.float64)
    h = O.round_to(x, "bf16")
    np.testing.assert_array_equal(hi, h)
    np.testing.assert_array_equal(lo, O.round_to(x - h, "bf16"))


@pytest.mark.parametrize("R,D,ldt", [(1000, 384, 1000), (33, 1024, 40), (4096, 384, 4096)])
def test_rmsnorm_t_and_planes(api, lib, R, D, ldt):
    rng = np.random.default_rng(R + D)
    x = rnd((R, D), "bf16", rng); w = rnd(D, "bf16", rng)
    dy = rng.normal(0, 1e-3, (R, D)).astype(np.float32).astype(np.float64)
    acc = rng.normal(0, 1e-3, (R, D)).astype(np.float32).astype(np.float64)
    eps = 1e-6
    X, W = dev(x, "bf16"), dev(w, "bf16")
    Y, Y2, YT = empty(R * D, "bf16"), empty(R * D, "bf16"), zeros(D * ldt, "bf16")
    api.sj_rmsnorm_fwd(None, X.p, BF, W.p, BF, Y.p, R, D, cf(eps))
    api.sj_rmsnorm_fwd_t(None, X.p, W.p, Y2.p, YT.p, ldt, R, D, cf(eps))
    DX, DW = empty(R * D), empty(D)
    Hn, Ln = empty(R * D, "bf16"), empty(R * D, "bf16")
    Ht, Lt = zeros(D * ldt, "bf16"), zeros(D * ldt, "bf16")
    wsb = empty(max(lib.sj_rmsnorm_bwd_p_workspace_bytes(R, D), 256), "u8")
    api.sj_rmsnorm_bwd_p(None, X.p, W.p, dev(dy).p, dev(acc).p, DX.p, DW.p, Hn.p, Ln.p, Ht.p, Lt.p, ldt, R, D,
                         cf(eps), wsb.p, wsb.nbytes)
    sync()
    y = Y.host().reshape(R, D)
    np.testing.assert_array_equal(Y2.host().reshape(R, D), y)   # same formula as the plain entry
    yt = YT.host().reshape(D, ldt)
    np.testing.assert_array_equal(yt[:, :R], y.T)
    assert not yt[:, R:].any()                                   # padding columns untouched
    dx, dw = O.rmsnorm_bwd(x, w, dy, eps, dx_acc=acc)
    dxd = DX.host().reshape(R, D)
    assert rel(dxd, dx) < 1e-5 and rel(DW.host(), dw) < 1e-5
    hi, lo = Hn.host().reshape(R, D), Ln.host().reshape(R, D)
    _check_planes(hi, lo, dxd)
    np.testing.assert_array_equal(Ht.host().reshape(D, ldt)[:, :R], hi.T)
    np.testing.assert_array_equal(Lt.host().reshape(D, ldt)[:, :R], lo.T)
    # planes are optional (the stage input's gradient): dx and dw are the same bits
    DX2, DW2 = empty(R * D), empty(D)
    api.sj_rmsnorm_bwd_p(None, X.p, W.p, dev(dy).p, dev(acc).p, DX2.p, DW2.p, None, None, None, None, 0, R, D,
                         cf(eps), wsb.p, wsb.nbytes)
    sync()
    np.testing.assert_array_equal(DX2.host(), DX.host())
    np.testing.assert_array_equal(DW2.host(), DW.host())


@pytest.mark.parametrize("B,T,HQ,HK", [(2, 256, 6, 2), (1, 200, 4, 4)])
def test_attention_t_and_planes(api, lib, B, T, HQ, HK):
    Dh = 64
    rng = np.random.default_rng(B * T + HQ + 5)
    M = B * T; N = HQ * Dh; KV = HK * Dh; NG = N + 2 * KV
    q = rnd((M, N), "bf16", rng); k = rnd((M, KV), "bf16", rng); v = rnd((M, KV), "bf16", rng)
    do = rng.normal(0, 1e-4, (M, N)).astype(np.float32).astype(np.float64)
    Q, K, V, DO = dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), dev(do)
    ldot = (M + 7) // 8 * 8
    O1, L1, O2, L2, OT = empty(M * N, "bf16"), empty(M * HQ), empty(M * N, "bf16"), empty(M * HQ), zeros(N * ldot, "bf16")
    print(f"[attention_t] B={B} T={T} HQ={HQ} HK={HK}", flush=True)
    api.sj_attention_fwd(None, Q.p, N, K.p, KV, V.p, KV, O1.p, N, L1.p, BF, B, T, HQ, HK, Dh, 0)
    api.sj_attention_fwd_t(None, Q.p, N, K.p, KV, V.p, KV, O2.p, N, L2.p, OT.p, ldot, B, T, HQ, HK, Dh)
    sync()
    o = O1.host().reshape(M, N)
    np.testing.assert_array_equal(O2.host().reshape(M, N), o)
    np.testing.assert_array_equal(L2.host(), L1.host())
    np.testing.assert_array_equal(OT.host().reshape(N, ldot)[:, :M], o.T)
    tab = empty(T * Dh)
    api.sj_rope_table(None, tab.p, T, Dh, cf(10000.0))
    dQ, dK, dV, De = empty(M * N), empty(M * KV), empty(M * KV), empty(M * HQ)
    api.sj_attention_bwd(None, Q.p, N, K.p, KV, V.p, KV, O1.p, N, L1.p, DO.p, N, dQ.p, N, dK.p, KV, dV.p, KV, De.p,
                         BF, B, T, HQ, HK, Dh, 0, tab.p)
    Gh, Gl, Th, Tl, De2 = (empty(M * NG, "bf16"), empty(M * NG, "bf16"), zeros(NG * ldot, "bf16"),
                           zeros(NG * ldot, "bf16"), empty(M * HQ))
    wsa = empty(max(lib.sj_attention_bwd_p_workspace_bytes(B, T, HQ, HK, Dh), 256), "u8")
    api.sj_attention_bwd_p(None, Q.p, N, K.p, KV, V.p, KV, O1.p, N, L1.p, DO.p, N, De2.p, B, T, HQ, HK, Dh, tab.p,
                           Gh.p, Gl.p, NG, Th.p, Tl.p, ldot, wsa.p, wsa.nbytes)
    sync()
    np.testing.assert_array_equal(De2.host(), De.host())
    ref = np.concatenate([dQ.host().reshape(M, N), dK.host().reshape(M, KV), dV.host().reshape(M, KV)], 1)
    hi, lo = Gh.host().reshape(M, NG), Gl.host().reshape(M, NG)
    _check_planes(hi[:, :N], lo[:, :N], ref[:, :N])              # dQ: same arithmetic as the fp32 entry
    # dK / dV: per-head partials summed over the group after the loop (a
    # different fp32 order than the fp32 entry's accumulators)
    assert rel((hi + lo)[:, N:], ref[:, N:]) < 1e-5
    assert np.all(np.abs(lo) <= 2.0 ** -8 * np.abs(hi) + 1e-38)
    np.testing.assert_array_equal(Th.host().reshape(NG, ldot)[:, :M], hi.T)
    np.testing.assert_array_equal(Tl.host().reshape(NG, ldot)[:, :M], lo.T)
    # and the oracle
    dq, dk, dv, _ = O.attention_bwd(q, k, v, o, L1.host(), do, B, T, HQ, HK, Dh, 0)
    dq = O.rope(dq, T, HQ, Dh, inverse=True); dk = O.rope(dk, T, HK, Dh, inverse=True)
    assert rel((hi + lo)[:, :N], dq) < 1e-4 and rel((hi + lo)[:, N:N + KV], dk) < 1e-4
    assert rel((hi + lo)[:, N + KV:], dv) < 1e-4


@pytest.mark.parametrize("B,T,HQ,HK,W", [(2, 256, 6, 2, 0), (1, 512, 4, 4, 0), (2, 128, 8, 1, 0), (2, 256, 4, 2, 128),
                                         (1, 320, 4, 1, 100), (2, 192, 4, 4, 32), (2, 256, 6, 2, 128),
                                         (1, 320, 3, 1, 100), (2, 512, 6, 2, 0), (1, 1024, 3, 1, 300),
                                         (1, 1024, 3, 1, 0)])
def test_attention_tt_against_row_path_and_oracle(api, lib, B, T, HQ, HK, W):
    """The step's MFMA-layout attention (q|k|v and dO planes in row
    orientation, transposed fragments by LDS transpose reads) against the
    fp32 row kernels and the FP64
    oracle on the same stored inputs; W > 0 is the local stages' sliding
    window (hierarchy.py:24,60,87), including windows that are not a
    multiple of the 64-key block and one shorter than a block."""
    Dh = 64
    rng = np.random.default_rng(B * T + HQ * 7 + HK)
    M = B * T; N = HQ * Dh; KV = HK * Dh; NG = N + 2 * KV
    ldq = NG + 8
    ldt = M + 8
    qkv = rnd((M, NG), "bf16", rng)
    QKV = dev(np.concatenate([qkv, np.zeros((M, ldq - NG))], 1), "bf16")
    q, k, v = qkv[:, :N], qkv[:, N:N + KV], qkv[:, N + KV:]
    print(f"[attention_tt] B={B} T={T} HQ={HQ} HK={HK} W={W}", flush=True)
    O1, L1 = empty(M * N, "bf16"), empty(M * HQ)
    api.sj_attention_fwd(None, QKV.p, ldq, QKV.at(N), ldq, QKV.at(N + KV), ldq, O1.p, N, L1.p, BF, B, T, HQ, HK, Dh, W)
    O2, L2, LT, OT = empty(M * N, "bf16"), empty(M * HQ), zeros(HQ * ldt), zeros(N * ldt, "bf16")
    api.sj_attention_fwd_tt(None, QKV.p, ldq, ldt, B, T, HQ, HK, Dh, W, O2.p, N, L2.p, LT.p, OT.p, ldt)
    sync()
    o1, o2 = O1.host().reshape(M, N), O2.host().reshape(M, N)
    # one storage ulp, plus the accumulation error of a result that cancels
    # (bounded through the same attention over |v|)
    o_abs, _ = O.attention_fwd(q, k, np.abs(v), B, T, HQ, HK, Dh, W)
    bad = np.abs(o2 - o1) > 2.0 ** -7 * np.abs(o1) + 2.0 ** -14 * o_abs + 1e-30
    if bad.any():
        r, c = np.nonzero(bad)
        print(f"[attention_tt] {bad.sum()} O elements beyond one ulp; rows%64 {np.unique(r % T % 64)[:20]} "
              f"pos {np.unique(r % T)[:10]} heads {np.unique(c // 64)} dims {np.unique(c % 64)[:20]}; "
              f"worst rel {np.max(np.abs(o2 - o1)[bad] / (np.abs(o1[bad]) + 1e-30)):.3e} rel(all) {rel(o2, o1):.3e}",
              flush=True)
    assert not bad.any(), "O beyond one bf16 ulp of the row kernel"
    assert rel(L2.host(), L1.host()) < 1e-6
    np.testing.assert_array_equal(LT.host().reshape(HQ, ldt)[:, :M], L2.host().reshape(M, HQ).T)
    np.testing.assert_array_equal(OT.host().reshape(N, ldt)[:, :M], o2.T)
    # backward from dO planes, against the fp32 row path on the same O and LSE
    do = rng.normal(0, 1e-4, (M, N)).astype(np.float32).astype(np.float64)
    dh = O.round_to(do, "bf16"); dl = O.round_to(do - dh, "bf16")
    DH_, DL_ = dev(dh, "bf16"), dev(dl, "bf16")
    tab = empty(T * Dh)
    api.sj_rope_table(None, tab.p, T, Dh, cf(10000.0))
    dof = dh + dl                                                  # the dO the planes carry
    DOF = dev(dof)
    dQ, dK, dV, De = empty(M * N), empty(M * KV), empty(M * KV), empty(M * HQ)
    api.sj_attention_bwd(None, QKV.p, ldq, QKV.at(N), ldq, QKV.at(N + KV), ldq, O2.p, N, L2.p, DOF.p, N, dQ.p, N,
                         dK.p, KV, dV.p, KV, De.p, BF, B, T, HQ, HK, Dh, W, tab.p)
    Gh, Gl, Th, Tl = empty(M * NG, "bf16"), empty(M * NG, "bf16"), zeros(NG * ldt, "bf16"), zeros(NG * ldt, "bf16")
    DT = zeros(HQ * ldt)
    # the workspace ends with the cut walks' meeting counters: zero before
    # the first call, and left zero by every call
    ws = zeros(max(lib.sj_attention_bwd_tt_workspace_bytes(B, T, HQ, HK, Dh), 256), "u8")
    ncnt = lib.sj_attention_bwd_tt_counter_bytes(B, HK)
    api.sj_attention_bwd_tt(None, QKV.p, ldq, ldt, O2.p, N, LT.p, DH_.p, DL_.p, N, DT.p,
                            B, T, HQ, HK, Dh, W, tab.p, Gh.p, Gl.p, NG, Th.p, Tl.p, ldt, ws.p, ws.nbytes)
    sync()
    assert rel(DT.host().reshape(HQ, ldt)[:, :M], De.host().reshape(M, HQ).T) < 1e-5
    ref = np.concatenate([dQ.host().reshape(M, N), dK.host().reshape(M, KV), dV.host().reshape(M, KV)], 1)
    hi, lo = Gh.host().reshape(M, NG), Gl.host().reshape(M, NG)
    got = hi + lo
    for name, sl in (("dq", slice(0, N)), ("dk", slice(N, N + KV)), ("dv", slice(N + KV, NG))):
        assert rel(got[:, sl], ref[:, sl]) < 1e-5, (name, rel(got[:, sl], ref[:, sl]))
    assert np.all(np.abs(lo) <= 2.0 ** -8 * np.abs(hi) + 1e-38)
    np.testing.assert_array_equal(Th.host().reshape(NG, ldt)[:, :M], hi.T)
    np.testing.assert_array_equal(Tl.host().reshape(NG, ldt)[:, :M], lo.T)
    # transposed outputs are optional (the row-layout dW step): same planes bit
    # for bit; with three query heads per KV head this is the grouped launch
    # (dK | dV summed inside the workgroup, no partials, no reduce pass), whose
    # walks longer than a cap are cut into parts added at the end (T 1024:
    # three-part walks): the same sums up to fp32 association, and the same
    # bits launch after launch
    G2h, G2l = empty(M * NG, "bf16"), empty(M * NG, "bf16")
    api.sj_attention_bwd_tt(None, QKV.p, ldq, ldt, O2.p, N, LT.p, DH_.p, DL_.p, N, DT.p, B, T, HQ, HK, Dh, W, tab.p,
                            G2h.p, G2l.p, NG, None, None, 0, ws.p, ws.nbytes)
    sync()
    if HQ == 3 * HK:
        g2 = G2h.host().reshape(M, NG) + G2l.host().reshape(M, NG)
        # hi + lo holds about 16 significant bits: a different fp32 sum may
        # round to the neighbouring pair
        assert rel(g2, got) < 1e-5, rel(g2, got)
        assert np.all(np.abs(g2 - got) <= 2.0 ** -14 * np.abs(got) + 2.0 ** -18 * np.abs(got).max())
        for _ in range(2):  # the cut walks' counters are back at zero after each launch
            G3h, G3l = empty(M * NG, "bf16"), empty(M * NG, "bf16")
            api.sj_attention_bwd_tt(None, QKV.p, ldq, ldt, O2.p, N, LT.p, DH_.p, DL_.p, N, DT.p, B, T, HQ, HK, Dh, W,
                                    tab.p, G3h.p, G3l.p, NG, None, None, 0, ws.p, ws.nbytes)
            sync()
            np.testing.assert_array_equal(G3h.host(), G2h.host())
            np.testing.assert_array_equal(G3l.host(), G2l.host())
        assert not ws.host()[ws.nbytes - ncnt:].any(), "meeting counters not back at zero"
        hi, lo = G2h.host().reshape(M, NG), G2l.host().reshape(M, NG)
        got = hi + lo
    else:
        np.testing.assert_array_equal(G2h.host().reshape(M, NG), hi)
        np.testing.assert_array_equal(G2l.host().reshape(M, NG), lo)
    dq, dk, dv, _ = O.attention_bwd(q, k, v, o2, L2.host(), dof, B, T, HQ, HK, Dh, W)
    dq = O.rope(dq, T, HQ, Dh, inverse=True); dk = O.rope(dk, T, HK, Dh, inverse=True)
    assert rel(got[:, :N], dq) < 1e-4 and rel(got[:, N:N + KV], dk) < 1e-4 and rel(got[:, N + KV:], dv) < 1e-4


def test_gemm_planes_split_out(api):
    rng = np.random.default_rng(21)
    M, N, K = 512, 384, 384
    a = rng.normal(0, 1e-3, (M, K)).astype(np.float32).astype(np.float64)
    ah = O.round_to(a, "bf16"); al = O.round_to(a - ah, "bf16")
    w = O.round_to(rng.normal(0, 0.05, (N, K)), "bf16")            # W^T [N][K]
    ldt = M + 8
    Ch, Cl, Th, Tl = empty(M * N, "bf16"), empty(M * N, "bf16"), zeros(N * ldt, "bf16"), zeros(N * ldt, "bf16")
    api.sj_gemm_planes_split_out(None, M, N, K, dev(ah, "bf16").p, dev(al, "bf16").p, K, dev(w, "bf16").p, K, Ch.p,
                                 Cl.p, N, Th.p, Tl.p, ldt, None, 0, None, 0)
    sync()
    hi, lo = Ch.host().reshape(M, N), Cl.host().reshape(M, N)
    assert rel(hi + lo, (ah + al) @ w.T) < 1e-5
    assert np.all(np.abs(lo) <= 2.0 ** -8 * np.abs(hi) + 1e-38)
    # deterministic: a second launch writes the same bits
    C2h, C2l = empty(M * N, "bf16"), empty(M * N, "bf16")
    api.sj_gemm_planes_split_out(None, M, N, K, dev(ah, "bf16").p, dev(al, "bf16").p, K, dev(w, "bf16").p, K, C2h.p,
                                 C2l.p, N, Th.p, Tl.p, ldt, None, 0, None, 0)
    sync()
    np.testing.assert_array_equal(C2h.host(), Ch.host())
    np.testing.assert_array_equal(C2l.host(), Cl.host())
    np.testing.assert_array_equal(Th.host().reshape(N, ldt)[:, :M], hi.T)
    # transposed outputs are optional: the normal planes are the same bits
    C3h, C3l = empty(M * N, "bf16"), empty(M * N, "bf16")
    api.sj_gemm_planes_split_out(None, M, N, K, dev(ah, "bf16").p, dev(al, "bf16").p, K, dev(w, "bf16").p, K, C3h.p,
                                 C3l.p, N, None, None, 0, None, 0, None, 0)
    sync()
    np.testing.assert_array_equal(C3h.host(), Ch.host())
    np.testing.assert_array_equal(C3l.host(), Cl.host())
    np.testing.assert_array_equal(Tl.host().reshape(N, ldt)[:, :M], lo.T)
    # Delta of the attention backward from the same epilogue: per row and
    # 64-column head, the sum of the stored planes times O (the planes are
    # unchanged by it)
    o = O.round_to(rng.normal(0, 1, (M, N)), "bf16")
    ldd = M + 16
    Dl, C4h, C4l = zeros(N // 64 * ldd, "f32"), empty(M * N, "bf16"), empty(M * N, "bf16")
    api.sj_gemm_planes_split_out(None, M, N, K, dev(ah, "bf16").p, dev(al, "bf16").p, K, dev(w, "bf16").p, K, C4h.p,
                                 C4l.p, N, None, None, 0, dev(o, "bf16").p, N, Dl.p, ldd)
    sync()
    np.testing.assert_array_equal(C4h.host(), Ch.host())
    np.testing.assert_array_equal(C4l.host(), Cl.host())
    want = ((hi + lo) * o).reshape(M, N // 64, 64).sum(-1).T
    got = Dl.host().reshape(N // 64, ldd)
    assert np.abs(got[:, :M] - want).max() <= 1e-5 * np.abs(want).max()
    assert np.all(got[:, M:] == 0)


def _raw(api, buf):
    """The buffer's bytes, without conversion."""
    out = np.empty(buf.nbytes, np.uint8)
    api.sj_download(ctypes.c_void_p(out.ctypes.data), buf.p, buf.nbytes)
    return out


def test_attention_tt_cut_walks_repeat_bits(api, lib):
    """The grouped backward at the bench's shape (cfg2: B 8, T 512, GQA 6/2),
    whose plan cuts the longest dK | dV walks into parts that meet through
    device-scope sums and a counter: 200 launches, alternating between two
    workspaces (each with its own counters), give the same bits every time,
    and both workspaces' counters are zero afterwards.  A stale read of a
    part's sum, or a counter shared between launches, would change the
    planes of a cut walk."""
    B, T, HQ, HK, W, Dh = 8, 512, 6, 2, 0, 64
    rng = np.random.default_rng(2024)
    M = B * T; N = HQ * Dh; KV = HK * Dh; NG = N + 2 * KV
    ldq, ldt = NG, M
    segs = (ctypes.c_uint32 * 128)()
    ncut = ctypes.c_int()
    n = lib.sj_attention_bwd_plan(T, W, B * HK, 256, segs, 128, ctypes.byref(ncut))
    assert n > 0 and ncut.value > 0, "the bench shape's plan must cut walks for this test to mean anything"
    qkv = rnd((M, NG), "bf16", rng)
    QKV = dev(qkv, "bf16")
    O2, L2, LT = empty(M * N, "bf16"), empty(M * HQ), zeros(HQ * ldt)
    api.sj_attention_fwd_tt(None, QKV.p, ldq, ldt, B, T, HQ, HK, Dh, W, O2.p, N, L2.p, LT.p, None, 0)
    do = rng.normal(0, 1e-4, (M, N)).astype(np.float32).astype(np.float64)
    dh = O.round_to(do, "bf16"); dl = O.round_to(do - dh, "bf16")
    DH_, DL_ = dev(dh, "bf16"), dev(dl, "bf16")
    tab = empty(T * Dh)
    api.sj_rope_table(None, tab.p, T, Dh, cf(10000.0))
    DT = zeros(HQ * ldt)
    wsb = lib.sj_attention_bwd_tt_workspace_bytes(B, T, HQ, HK, Dh)
    ncnt = lib.sj_attention_bwd_tt_counter_bytes(B, HK)
    wss = [zeros(wsb, "u8"), zeros(wsb, "u8")]
    Gh, Gl = empty(M * NG, "bf16"), empty(M * NG, "bf16")
    first = None
    print(f"[attention_tt repeat] B={B} T={T} HQ={HQ} HK={HK}: {n} pieces, {ncut.value} cut walks per pair",
          flush=True)
    for it in range(200):
        ws = wss[it & 1]
        api.sj_attention_bwd_tt(None, QKV.p, ldq, ldt, O2.p, N, LT.p, DH_.p, DL_.p, N, DT.p, B, T, HQ, HK, Dh, W,
                                tab.p, Gh.p, Gl.p, NG, None, None, 0, ws.p, ws.nbytes)
        sync()
        got = (_raw(api, Gh), _raw(api, Gl))
        if first is None:
            first = got
            assert np.any(got[0]), "planes written"
        else:
            assert np.array_equal(got[0], first[0]) and np.array_equal(got[1], first[1]), f"bits differ at launch {it}"
        if it % 50 == 49:
            print(f"[attention_tt repeat] {it + 1} launches identical", flush=True)
    for ws in wss:
        assert not _raw(api, ws)[wsb - ncnt:].any(), "meeting counters not back at zero"
