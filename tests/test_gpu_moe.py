"""Parity of the MoE FFN (routing, device-side pack, grouped expert GEMMs,
combine and their backward) against the FP64 oracle, through the C ABI.

Routing ids, the pack (tokens, slots, counts) and the gather are checked
bit-exactly (the reference rule applied to the device's stored logits).
Floating-point outputs are checked op by op on the device-stored inputs, and
the gradients end to end against the FP64 backward conditioned on the
device-stored forward activations (as the reference's own checks condition
on stored operands)."""
import ctypes

import numpy as np
import pytest

from oracle import moe
from oracle import oracle as O
from tests.gpu_util import assert_stored_close, dev, empty, rel, sync, zeros

pytestmark = pytest.mark.gpu

BF, F32 = 4, 0


@pytest.fixture(scope="module")
def api():
    from sejong_amd import _native as N
    N.load()
    return N.api


@pytest.fixture(scope="module")
def lib():
    from sejong_amd import _native as N
    return N.load()


def _split_ok(hi, lo, x):
    x = np.asarray(x, np.float32).astype(np.float64)
    h = O.round_to(x, "bf16")
    np.testing.assert_array_equal(hi, h)
    np.testing.assert_array_equal(lo, O.round_to(x - h, "bf16"))


MOE_CASES = [
    # M, d, E, F, K
    (4096, 512, 8, 1024, 2),   # cfg4 layer shape
    (300, 64, 5, 96, 3),       # ragged: partial tiles, empty-ish experts, K=3 ordering
]


@pytest.mark.parametrize("M,d,E,F,K", MOE_CASES)
def test_moe_ffn_forward_backward(api, lib, M, d, E, F, K):
    rng = np.random.default_rng(M + d + E)
    print(f"[moe] M={M} d={d} E={E} F={F} K={K}", flush=True)
    z = O.round_to(rng.normal(0, 1, (M, d)), "bf16")
    x1 = O.round_to(rng.normal(0, 1, (M, d)), "bf16")
    wr = O.round_to(rng.normal(0, d ** -0.5, (d, E)), "bf16")
    wg = O.round_to(rng.normal(0, 0.05, (E, d, F)), "bf16")
    wu = O.round_to(rng.normal(0, 0.05, (E, d, F)), "bf16")
    wd = O.round_to(rng.normal(0, 0.05, (E, F, d)), "bf16")
    experts = [(wg[e], wu[e], wd[e]) for e in range(E)]
    cap = lib.sj_route_pack_capacity(M * K, E)
    assert cap % 64 == 0 and cap >= M * K + 63 * E - 63

    # ---------------------------------------------------------- forward
    Z, WR, X1 = dev(z, "bf16"), dev(wr, "bf16"), dev(x1, "bf16")
    wgu_t = np.concatenate([wg.transpose(0, 2, 1), wu.transpose(0, 2, 1)], axis=1)   # [E][2F][d]
    wgu = np.concatenate([wg, wu], axis=2)                                            # [E][d][2F]
    WGUT, WGU = dev(wgu_t, "bf16"), dev(wgu, "bf16")
    WDT, WD = dev(wd.transpose(0, 2, 1), "bf16"), dev(wd, "bf16")                     # [E][d][F], [E][F][d]
    LOG, IDS, WTS = empty(M * E, "bf16"), empty(M * K, "i32"), empty(M * K)
    api.sj_router_topk(None, Z.p, d, WR.p, d, M, E, K, LOG.p, IDS.p, WTS.p)
    TOK, SLT = zeros(E * M * K, "i32"), zeros(E * M * K, "i32")
    CNT, OFF, PS, PP = empty(E, "i32"), empty(E + 1, "i32"), zeros(cap, "i32"), empty(M * K, "i32")
    api.sj_route_pack(None, IDS.p, M, K, E, TOK.p, SLT.p, CNT.p, OFF.p, PS.p, PP.p, cap)
    ZP, ZPT = zeros(cap * d, "bf16"), zeros(d * cap, "bf16")
    api.sj_moe_gather(None, Z.p, d, d, PS.p, K, cap, ZP.p, ZPT.p, cap)
    G, U, H, HT = zeros(cap * F, "bf16"), zeros(cap * F, "bf16"), zeros(cap * F, "bf16"), zeros(F * cap, "bf16")
    api.sj_moe_gate_up_fwd(None, OFF.p, E, cap, ZP.p, d, d, WGUT.p, WGUT.at(F * d), d, 2 * F * d, F, G.p, U.p, H.p,
                           F, HT.p, cap)
    YP = zeros(cap * d, "bf16")
    api.sj_moe_down_fwd(None, OFF.p, E, cap, H.p, F, F, WDT.p, F, d * F, d, YP.p, d)
    OUT = empty(M * d, "bf16")
    api.sj_moe_combine(None, YP.p, d, d, IDS.p, PP.p, WTS.p, M, K, X1.p, d, OUT.p, d)
    # the row-only gather (16-byte chunks) and the combine through its
    # 2-column path (an output stride that is not a multiple of 8) give the
    # same bits as the forms above
    ZP2 = zeros(cap * d, "bf16")
    api.sj_moe_gather(None, Z.p, d, d, PS.p, K, cap, ZP2.p, None, cap)
    OUT2 = zeros(M * (d + 2), "bf16")
    api.sj_moe_combine(None, YP.p, d, d, IDS.p, PP.p, WTS.p, M, K, X1.p, d, OUT2.p, d + 2)
    sync()
    np.testing.assert_array_equal(ZP2.host(), ZP.host())
    np.testing.assert_array_equal(OUT2.host().reshape(M, d + 2)[:, :d], OUT.host().reshape(M, d))

    logits = LOG.host().reshape(M, E)
    assert_stored_close(logits, z @ wr, "bf16", "logits", terms=np.abs(z) @ np.abs(wr))
    ids, w = IDS.host().reshape(M, K), WTS.host().reshape(M, K)
    ids_ref, w_ref = O.route_topk(logits.astype(np.float32), K)
    np.testing.assert_array_equal(ids, ids_ref)                       # bit-exact routing
    assert rel(w, w_ref) < 1e-6
    tokens_ref, slots_ref, counts_ref = O.route_pack(ids, E)
    counts, off = CNT.host(), OFF.host()
    np.testing.assert_array_equal(counts, counts_ref)
    pad = (counts + 63) // 64 * 64
    np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(pad)]))
    tok, slt = TOK.host().reshape(E, M * K), SLT.host().reshape(E, M * K)
    pslot, ppos = PS.host(), PP.host()
    for e in range(E):
        c = counts[e]
        np.testing.assert_array_equal(tok[e, :c], tokens_ref[e, :c])
        np.testing.assert_array_equal(slt[e, :c], slots_ref[e, :c])
        np.testing.assert_array_equal(pslot[off[e]:off[e] + c], slots_ref[e, :c])
        assert np.all(pslot[off[e] + c:off[e + 1]] == -1)
    assert np.all(pslot[off[E]:] == -1)
    np.testing.assert_array_equal(pslot[ppos], np.arange(M * K))
    zp = ZP.host().reshape(cap, d)
    ref_zp = np.where(pslot[:, None] >= 0, z[np.maximum(pslot, 0) // K], 0.0)
    np.testing.assert_array_equal(zp, ref_zp)
    np.testing.assert_array_equal(ZPT.host().reshape(d, cap), zp.T)

    g, u, h = (B.host().reshape(cap, F) for B in (G, U, H))
    yp = YP.host().reshape(cap, d)
    real = pslot >= 0
    inside = np.arange(cap) < off[E]          # rows past the last segment are never launched or read
    for X in (g, u, h, yp):
        assert not X[~real & inside].any()                            # segment padding rows stay zero
    np.testing.assert_array_equal(HT.host().reshape(F, cap)[:, :off[E]], h[:off[E]].T)
    for e in range(E):
        r = slice(off[e], off[e] + counts[e])
        if counts[e] == 0:
            continue
        a = np.abs(zp[r])
        assert_stored_close(g[r], zp[r] @ wg[e], "bf16", f"g[{e}]", terms=a @ np.abs(wg[e]))
        assert_stored_close(u[r], zp[r] @ wu[e], "bf16", f"u[{e}]", terms=a @ np.abs(wu[e]))
        assert_stored_close(h[r], O.swiglu_fwd(g[r], u[r]), "bf16", f"h[{e}]")
        assert_stored_close(yp[r], h[r] @ wd[e], "bf16", f"y[{e}]", terms=np.abs(h[r]) @ np.abs(wd[e]))
    wflat = w.ravel()
    comb = np.zeros((M, d))
    np.add.at(comb, np.arange(M * K) // K, wflat[:, None] * yp[ppos])
    assert_stored_close(OUT.host(), x1 + comb, "bf16", "combine + residual", ulps=2,
                        terms=2 ** 9 * np.abs(comb) + np.abs(comb))

    # --------------------------------------------------------- backward
    dup = rng.normal(0, 1e-3, (M, d)).astype(np.float32).astype(np.float64)
    acc = rng.normal(0, 1e-3, (M, d)).astype(np.float32).astype(np.float64)
    DUP, ACC = dev(dup), dev(acc)
    DXH, DXL, DXTH, DXTL = (zeros(cap * d, "bf16") for _ in range(4))
    DWT = empty(M * K)
    api.sj_moe_combine_bwd(None, YP.p, d, d, PS.p, WTS.p, K, cap, DUP.p, d, DXH.p, DXL.p, DXTH.p, DXTL.p, cap, DWT.p)
    # the rows-only form (one wave per packed row, 8 columns per lane): the
    # same planes bit for bit; its dw sums in another order (checked below)
    DXH8, DXL8, DWT8 = zeros(cap * d, "bf16"), zeros(cap * d, "bf16"), empty(M * K)
    api.sj_moe_combine_bwd(None, YP.p, d, d, PS.p, WTS.p, K, cap, DUP.p, d, DXH8.p, DXL8.p, None, None, cap, DWT8.p)
    DGH, DGL, DGTH, DGTL = (zeros(cap * 2 * F, "bf16") for _ in range(4))
    api.sj_moe_down_bwd_swiglu_p(None, OFF.p, E, cap, DXH.p, DXL.p, d, d, WD.p, d, F * d, F, G.p, U.p, F, DGH.p,
                                 DGL.p, 2 * F, DGTH.p, DGTL.p, cap)
    DGH2, DGL2 = (zeros(cap * 2 * F, "bf16") for _ in range(2))
    api.sj_moe_down_bwd_swiglu_p(None, OFF.p, E, cap, DXH.p, DXL.p, d, d, WD.p, d, F * d, F, G.p, U.p, F, DGH2.p,
                                 DGL2.p, 2 * F, None, None, cap)
    DWD = empty(E * F * d)
    api.sj_moe_gemm_dw(None, OFF.p, E, cap, F, d, HT.p, cap, DXTH.p, DXTL.p, cap, DWD.p, d, F * d)
    DZP = zeros(cap * d)
    api.sj_moe_gemm_rows(None, OFF.p, E, cap, d, 2 * F, DGH.p, DGL.p, 2 * F, WGU.p, 2 * F, d * 2 * F, DZP.p, d, 0)
    DWGU = empty(E * d * 2 * F)
    api.sj_moe_gemm_dw(None, OFF.p, E, cap, d, 2 * F, ZPT.p, cap, DGTH.p, DGTL.p, cap, DWGU.p, 2 * F, d * 2 * F)
    # the same dW from row-layout operands (packed h / inputs and the normal planes)
    DWD2, DWGU2 = empty(E * F * d), empty(E * d * 2 * F)
    api.sj_moe_gemm_dw_tn(None, OFF.p, E, cap, F, d, H.p, F, DXH.p, DXL.p, d, DWD2.p, d, F * d)
    api.sj_moe_gemm_dw_tn(None, OFF.p, E, cap, d, 2 * F, ZP.p, d, DGH.p, DGL.p, 2 * F, DWGU2.p, 2 * F, d * 2 * F)
    DZ, DLOG = empty(M * d), empty(M * E)
    api.sj_moe_gather_bwd(None, DZP.p, d, d, IDS.p, PP.p, WTS.p, LOG.p, DWT.p, WR.p, M, K, E, ACC.p, d, DZ.p, d,
                          DLOG.p)
    DWR = empty(d * E)
    ws = empty(max(lib.sj_gemm_workspace_bytes(d, E, M), 256), "u8")
    api.sj_gemm(None, 1, 0, d, E, M, Z.p, BF, d, DLOG.p, F32, E, DWR.p, F32, E, 0, ws.p, ws.nbytes)
    sync()

    # per-op checks on the stored operands
    dxh, dxl = DXH.host().reshape(cap, d), DXL.host().reshape(cap, d)
    dx_val = np.where(real[:, None], dup[np.maximum(pslot, 0) // K] * wflat[np.maximum(pslot, 0)][:, None], 0.0)
    _split_ok(dxh, dxl, dx_val.astype(np.float32))
    np.testing.assert_array_equal(DXTH.host().reshape(d, cap), dxh.T)
    np.testing.assert_array_equal(DXTL.host().reshape(d, cap), dxl.T)
    dgh, dgl = DGH.host().reshape(cap, 2 * F), DGL.host().reshape(cap, 2 * F)
    n = off[E]
    np.testing.assert_array_equal(DGTH.host().reshape(2 * F, cap)[:, :n], dgh[:n].T)
    np.testing.assert_array_equal(DGTL.host().reshape(2 * F, cap)[:, :n], dgl[:n].T)
    # the row-plane epilogue (no transposed outputs) writes the same planes
    np.testing.assert_array_equal(DGH2.host().reshape(cap, 2 * F)[:n], dgh[:n])
    np.testing.assert_array_equal(DGL2.host().reshape(cap, 2 * F)[:n], dgl[:n])

    # end to end, conditioned on the device-stored forward activations
    per = []
    for e in range(E):
        r = slice(off[e], off[e] + counts[e])
        tk = tokens_ref[e, :counts[e]].astype(np.int64)
        per.append(dict(tokens=tk, slots=slots_ref[e, :counts[e]].astype(np.int64), x=z[tk], g=g[r], u=u[r], h=h[r],
                        y=yp[r]))
    acts = dict(logits=logits, ids=ids, w=w, per=per)
    dz_ref, dwr_ref, grads_ref, dwts_ref, dlog_ref = moe.moe_backward(z, wr, experts, acts, dup)
    assert rel(DWT.host(), dwts_ref) < 1e-5
    assert rel(DWT8.host(), dwts_ref) < 1e-5
    np.testing.assert_array_equal(DXH8.host(), DXH.host())
    np.testing.assert_array_equal(DXL8.host(), DXL.host())
    assert rel(DLOG.host(), dlog_ref) < 1e-4
    dwd = DWD.host().reshape(E, F, d)
    dwgu = DWGU.host().reshape(E, d, 2 * F)
    worst = 0.0
    for e in range(E):
        if counts[e] == 0:
            assert not dwd[e].any() and not dwgu[e].any()
            continue
        for got, ref in ((dwgu[e][:, :F], grads_ref[e][0]), (dwgu[e][:, F:], grads_ref[e][1]), (dwd[e], grads_ref[e][2])):
            worst = max(worst, rel(got, ref))
    assert worst < 1e-4, worst
    assert rel(DWD2.host(), DWD.host()) < 1e-6 and rel(DWGU2.host(), DWGU.host()) < 1e-6
    assert rel(DZ.host(), acc + dz_ref) < 1e-4
    assert rel(DWR.host(), dwr_ref) < 1e-4
    print(f"[moe] worst expert dW rel {worst:.2e}", flush=True)


def test_route_topk_and_backward_entries(api):
    """The standalone Engine::route_topk / route_topk_backward entries, on
    fp32 and bf16 logits, with ties (lowest index wins)."""
    rng = np.random.default_rng(5)
    R, E, K = 1000, 8, 2
    x = O.round_to(rng.normal(0, 1, (R, E)), "bf16")
    x[:10, 3] = x[:10, 5] = 4.0                                       # exact ties
    for dt, code in (("bf16", BF), ("f32", F32)):
        X, IDS, W = dev(x, dt), empty(R * K, "i32"), empty(R * K)
        api.sj_route_topk(None, X.p, code, R, E, K, IDS.p, W.p)
        dy = rng.normal(0, 1, (R, K)).astype(np.float32).astype(np.float64)
        DX = empty(R * E)
        api.sj_route_topk_bwd(None, X.p, code, IDS.p, W.p, dev(dy).p, DX.p, R, E, K)
        sync()
        ids, w = O.route_topk(x.astype(np.float32), K)
        np.testing.assert_array_equal(IDS.host().reshape(R, K), ids)
        assert np.all(ids[:10, 0] == 3) and np.all(ids[:10, 1] == 5)
        assert rel(W.host(), w) < 1e-6
        assert rel(DX.host(), O.route_topk_bwd(x.astype(np.float32), ids, W.host().reshape(R, K), dy)) < 1e-5


@pytest.mark.parametrize("E,K", [(2, 1), (3, 2), (8, 2), (16, 4), (32, 8)])
def test_route_pack_all_expert_counts(api, lib, E, K):
    """The device pack (every template width and the 32-expert form) against
    the reference's stable slot-order pack (hierarchy.py:212-225) on ids
    with empty and full experts."""
    rng = np.random.default_rng(E * 10 + K)
    M = 2000
    ids = np.stack([rng.permutation(E)[:K] for _ in range(M)]).astype(np.int32)
    ids[:, 0] = np.where(rng.random(M) < 0.5, 0, ids[:, 0])            # a crowded expert (the pack is per slot)
    if E > 2:
        ids[ids == E - 1] = E - 2 if K == 1 else ids[ids == E - 1]        # expert E-1 may stay empty (K = 1)
    S = M * K
    cap = lib.sj_route_pack_capacity(S, E)
    IDS = dev(ids.ravel(), "i32")
    TOK, SLT = empty(E * S, "i32"), empty(E * S, "i32")
    CNT, OFF, PS, PP = empty(E, "i32"), empty(E + 1, "i32"), empty(cap, "i32"), empty(S, "i32")
    print(f"[route_pack] E={E} K={K} S={S}", flush=True)
    api.sj_route_pack(None, IDS.p, M, K, E, TOK.p, SLT.p, CNT.p, OFF.p, PS.p, PP.p, cap)
    sync()
    tokens_ref, slots_ref, counts_ref = O.route_pack(ids, E)
    counts, off = CNT.host(), OFF.host()
    np.testing.assert_array_equal(counts, counts_ref)
    pad = (counts_ref + 63) // 64 * 64
    np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(pad)]))
    tok, slt, pslot = TOK.host().reshape(E, S), SLT.host().reshape(E, S), PS.host()
    for e in range(E):
        c = counts[e]
        np.testing.assert_array_equal(tok[e, :c], tokens_ref[e, :c])
        np.testing.assert_array_equal(slt[e, :c], slots_ref[e, :c])
        np.testing.assert_array_equal(pslot[off[e]:off[e] + c], slots_ref[e, :c])
        assert np.all(pslot[off[e] + c:off[e + 1]] == -1)
    assert np.all(pslot[off[E]:] == -1)
    np.testing.assert_array_equal(pslot[PP.host()], np.arange(S))


def test_gather_bwd_vector_form_is_bit_exact(api, lib):
    """The 16-byte gather/route backward equals the per-column kernel bit
    for bit (same per-column order); an odd dz stride selects the latter."""
    rng = np.random.default_rng(77)
    M, d, E, K = 1000, 256, 8, 2
    cap = lib.sj_route_pack_capacity(M * K, E)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(M)]).astype(np.int32)
    IDS = dev(ids.ravel(), "i32")
    CNT, OFF, PS, PP = empty(E, "i32"), empty(E + 1, "i32"), empty(cap, "i32"), empty(M * K, "i32")
    api.sj_route_pack(None, IDS.p, M, K, E, None, None, CNT.p, OFF.p, PS.p, PP.p, cap)
    logits = O.round_to(rng.normal(0, 1, (M, E)), "bf16")
    _, w = O.route_topk(logits.astype(np.float32), K)
    dxp = rng.normal(0, 1e-3, (cap, d)).astype(np.float32).astype(np.float64)
    acc = rng.normal(0, 1e-3, (M, d)).astype(np.float32).astype(np.float64)
    wr = O.round_to(rng.normal(0, d ** -0.5, (d, E)), "bf16")
    dwt = rng.normal(0, 1e-2, (M, K)).astype(np.float32).astype(np.float64)
    args = (dev(dxp).p, d, d, IDS.p, PP.p, dev(w).p, dev(logits, "bf16").p, dev(dwt).p, dev(wr, "bf16").p, M, K, E,
            dev(acc).p, d)
    DZ, DL = empty(M * d), empty(M * E)
    api.sj_moe_gather_bwd(None, *args, DZ.p, d, DL.p)
    DZ2, DL2 = empty(M * (d + 1)), empty(M * E)
    api.sj_moe_gather_bwd(None, *args, DZ2.p, d + 1, DL2.p)
    sync()
    np.testing.assert_array_equal(DZ.host().reshape(M, d), DZ2.host().reshape(M, d + 1)[:, :d])
    np.testing.assert_array_equal(DL.host(), DL2.host())
