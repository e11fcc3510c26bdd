"""Parity of the parameter-VJP path (indices, CGS2 basis, prepare,
coefficients, factored gradient / update / norm) through the C ABI.

The first test restates the reference's own check program
(crates/sejong-gpu/examples/parameter_vjp_check.rs) on its default shape:
the selected columns and rows must equal the exact CPU generator bit for
bit, and the factored gradient, norm and SGD update must meet its
shape-derived roundoff budget against FP64 computed from the device basis
Q (the reference conditions on the device Q the same way, :111-131)."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from oracle import pvjp
from tests.gpu_util import Dev, dev, empty, rel, sync, zeros

pytestmark = pytest.mark.gpu

BF, F32 = 4, 0
cf = ctypes.c_float


@pytest.fixture(scope="module")
def N():
    from sejong_amd import _native as N
    N.load()
    return N


def _planes(x):
    x = np.asarray(x, np.float32).astype(np.float64)
    h = O.round_to(x, "bf16")
    return h, O.round_to(x - h, "bf16")


def _prepare(N, X, Y, rank, frac, block_rows, seed, ydtype="f32"):
    """indices + basis + prepare on device; returns a dict of host copies and
    device buffers."""
    api, lib = N.api, N.load()
    n, a = X.shape
    b = Y.shape[1]
    R, blocks, S = pvjp.budget(rank, frac, block_rows, n, a, b)
    k = S * block_rows
    SCR, COL = empty(b + blocks, "i32"), empty(R, "i32")
    ROWS, MAP = empty(k, "i32"), empty(a, "i32")
    api.sj_pvjp_indices(None, seed, a, b, blocks, S, R, block_rows, SCR.p, COL.p, ROWS.p, MAP.p)
    Q = empty(n * R)
    eps = lib.sj_pvjp_basis_tolerance(n, R)
    YD = dev(Y, ydtype)
    wsb = empty(max(lib.sj_pvjp_basis_workspace_bytes(n, R), 256), "u8")
    api.sj_pvjp_basis(None, YD.p, BF if ydtype == "bf16" else F32, b, n, COL.p, R, cf(eps), Q.p, wsb.p, wsb.nbytes)
    n8 = (n + 7) // 8 * 8
    xt = np.zeros((a, n8)); xt[:, :n] = X.T
    XT = dev(xt, "bf16")
    LEFT, E = empty(a * R), empty((R + k) * n8)
    EH, EL = empty((R + k) * n8, "bf16"), empty((R + k) * n8, "bf16")
    ws = empty(max(lib.sj_pvjp_prepare_workspace_bytes(a, n, R), 256), "u8")
    inverse = float(np.float32(blocks / S))
    api.sj_pvjp_prepare(None, XT.p, n8, a, n, Q.p, R, ROWS.p, k, cf(inverse), LEFT.p, E.p, EH.p, EL.p, n8,
                        ws.p, ws.nbytes)
    sync()
    return dict(R=R, blocks=blocks, S=S, k=k, n8=n8, eps=eps, cols=COL.host(), rows=ROWS.host(), map=MAP.host(),
                q=Q.host().reshape(n, R), left=LEFT.host().reshape(a, R), e=E.host().reshape(R + k, n8),
                eh=EH.host().reshape(R + k, n8), el=EL.host().reshape(R + k, n8), EH=EH, EL=EL, LEFT=LEFT, MAP=MAP,
                inverse=inverse, Q=Q, ROWS=ROWS)


def _coefficients(N, P, D):
    api, lib = N.api, N.load()
    n, b = D.shape
    n8, rk = P["n8"], P["R"] + P["k"]
    dt = np.zeros((b, n8)); dt[:, :n] = D.T
    dh, dl = _planes(dt)
    DH, DL = dev(dh, "bf16"), dev(dl, "bf16")
    C = empty(rk * b)
    ws = empty(max(lib.sj_pvjp_vjp_workspace_bytes(rk, b, n), 256), "u8")
    api.sj_pvjp_vjp(None, P["EH"].p, P["EL"].p, n8, rk, n, DH.p, DL.p, n8, b, C.p, b, ws.p, ws.nbytes)
    sync()
    return C


def _pack(N, params, terms):
    """params: (W Dev, dense Dev|None, rows, cols, decay, term_begin, term_count);
    terms: (left Dev, right ptr, tail ptr, map Dev, rank, scale)."""
    api, lib = N.api, N.load()
    PA = (N.FactoredParam * len(params))()
    for i, (w, dense, r, c, decay, tb, tc) in enumerate(params):
        PA[i] = N.FactoredParam(w.ptr, dense.ptr if dense else None, r, c, decay, tb, tc)
    TA = (N.FactoredTerm * max(len(terms), 1))()
    for i, (left, right, tail, fmap, rank, scale) in enumerate(terms):
        TA[i] = N.FactoredTerm(left.ptr, right.value, tail.value, fmap.ptr, rank, scale, 0)
    nbytes = lib.sj_factored_meta_bytes(PA, len(params), len(terms))
    host = np.zeros(nbytes, np.uint8)
    tiles = ctypes.c_long()
    api.sj_factored_pack(PA, len(params), TA, len(terms), ctypes.c_void_p(host.ctypes.data), nbytes,
                         ctypes.byref(tiles))
    meta = Dev(nbytes, "u8").upload(host)
    return meta, tiles.value


def test_reference_check_program(N):
    api = N.api
    n, a, b, rank, frac, block_rows = 67, 71, 97, 33, 0.4, 16
    rng = np.random.default_rng(42)
    X = O.round_to(rng.normal(0, 1, (n, a)), "bf16")
    W = rng.normal(0, 1, (a, b)).astype(np.float32).astype(np.float64) / np.sqrt(a)
    W = W.astype(np.float32).astype(np.float64)
    D = (rng.normal(0, 1, (n, b)) / n).astype(np.float32).astype(np.float64)
    Y = (X @ W).astype(np.float32).astype(np.float64)
    host_rng = O.Rng(42)
    seed = host_rng.next_u64()                      # prepare_parameter_vjp_reusing draws once (:189)
    print(f"[pvjp] check shape n={n} a={a} b={b} rank={rank}", flush=True)
    P = _prepare(N, X, Y, rank, frac, block_rows, seed)
    R, blocks, S, k = P["R"], P["blocks"], P["S"], P["k"]
    cols_ref, rows_ref, map_ref = pvjp.indices(seed, a, b, blocks, S, R, block_rows)
    np.testing.assert_array_equal(P["cols"], cols_ref)
    np.testing.assert_array_equal(P["rows"], rows_ref)
    np.testing.assert_array_equal(P["map"], map_ref)
    # basis: orthonormal within the check's budget, same span as FP64 CGS2
    ops = 2 * n * rank + 2 * n + rank
    tol = ops * 2.0 ** -23 / (1 - ops * 2.0 ** -23)
    q = P["q"]
    assert np.abs(q.T @ q - np.eye(R)).max() < tol
    q64 = pvjp.basis(Y, cols_ref, P["eps"])
    assert np.abs(q @ q.T - q64 @ q64.T).max() < 1e-4
    # prepare, conditioned on the device Q
    A_ref, E_ref = pvjp.prepare(X, q, rows_ref, blocks, S)
    assert rel(P["left"], A_ref) < 1e-5
    assert rel(P["e"][:, :n], E_ref) < 1e-5
    assert not P["e"][:, n:].any()
    _h, _l = _planes(P["e"])
    np.testing.assert_array_equal(P["eh"], _h)
    np.testing.assert_array_equal(P["el"], _l)
    # coefficients and the materialised factored gradient
    C = _coefficients(N, P, D)
    coeff = C.host().reshape(R + k, b)
    assert rel(coeff, (_h + _l)[:, :n] @ D) < 1e-5
    right = ctypes.c_void_p(C.ptr)
    tail = ctypes.c_void_p(C.ptr + R * b * 4)
    G = zeros(a * b)
    meta, tiles = _pack(N, [(G, None, a, b, 1, 0, 1)], [(P["LEFT"], right, tail, P["MAP"], R, 1.0)])
    api.sj_factored_apply(None, meta.p, tiles, 0, cf(0), cf(0), None)
    sync()
    got = G.host().reshape(a, b)
    # expected as the check builds it: left right + the selected rows' residual
    qd = q.astype(np.float64)
    left = X.T @ qd
    expected = left @ (qd.T @ D)
    projected = qd @ left.T
    inv = blocks / S
    for row in P["rows"]:
        if row >= 0:
            expected[row] += (X[:, row] - projected[:, row]) @ D * inv
    rel_sq = np.sum((got - expected) ** 2) / np.sum(expected ** 2)
    assert rel_sq < tol * tol, (rel_sq, tol * tol)

    # second term (rank/2), dense W, accumulation scales 0.5 / -0.25: norm and update
    P2 = _prepare(N, X, Y, (rank + 1) // 2, frac, block_rows, host_rng.next_u64())
    C2 = _coefficients(N, P2, D)
    R2 = P2["R"]
    q2 = P2["q"]
    a2 = X.T @ q2
    expected2 = a2 @ (q2.T @ D)
    proj2 = q2 @ a2.T
    for row in P2["rows"]:
        if row >= 0:
            expected2[row] += (X[:, row] - proj2[:, row]) @ D * inv
    Wd = dev(W)
    Wdense = dev(W)                                   # dense term = a copy of W (Engine::scale(w, 1))
    terms = [(P["LEFT"], right, tail, P["MAP"], R, 0.5),
             (P2["LEFT"], ctypes.c_void_p(C2.ptr), ctypes.c_void_p(C2.ptr + R2 * b * 4), P2["MAP"], R2, -0.25)]
    meta, tiles = _pack(N, [(Wd, Wdense, a, b, 1, 0, 2)], terms)
    part, out = empty(tiles, "f64"), empty(1, "f64")
    api.sj_factored_apply(None, meta.p, tiles, 2, cf(0), cf(0), part.p)
    api.sj_sum_f64(None, part.p, tiles, out.p)
    sync()
    g_exp = W + 0.5 * expected - 0.25 * expected2
    ref_norm = np.sqrt(np.sum(g_exp ** 2))
    assert abs(np.sqrt(out.host()[0]) - ref_norm) <= tol * ref_norm
    lr, clip, wd = 0.01, 0.7, 0.02
    LR = float(np.float32(np.float32(lr) * np.float32(clip)))
    DEC = float(np.float32(np.float32(lr) * np.float32(wd)))
    api.sj_factored_apply(None, meta.p, tiles, 1, cf(LR), cf(DEC), None)
    sync()
    w_exp = pvjp.factored_update(W, g_exp, lr, clip, wd, True)
    rel_sq = np.sum((Wd.host().reshape(a, b) - w_exp) ** 2) / np.sum(w_exp ** 2)
    assert rel_sq < tol * tol


def test_large_gradient_update_is_finite(N):
    """parameter_vjp_check.rs:237-253: dense f32::MAX/2 gradient, lr 2^-10."""
    api = N.api
    big = np.float32(np.finfo(np.float32).max) / np.float32(2)
    Z, L = zeros(16), dev(np.full(16, big, np.float32))
    meta, tiles = _pack(N, [(Z, L, 4, 4, 1, 0, 0)], [])
    part, out = empty(tiles, "f64"), empty(1, "f64")
    api.sj_factored_apply(None, meta.p, tiles, 2, cf(0), cf(0), part.p)
    api.sj_sum_f64(None, part.p, tiles, out.p)
    api.sj_factored_apply(None, meta.p, tiles, 1, cf(2.0 ** -10), cf(0.0), None)
    sync()
    assert np.sqrt(out.host()[0]) > float(np.finfo(np.float32).max)
    assert np.all(Z.host() == -float(np.float32(np.finfo(np.float32).max) / np.float32(2048)))


@pytest.mark.parametrize("seed,a,b,blocks,S,R,group", [
    (1, 1024, 5504, 32, 4, 16, 32), (2 ** 63 + 12345, 71, 97, 5, 2, 33, 16), (7, 100, 64, 4, 3, 64, 32),
    (123456789, 5000, 3000, 157, 50, 20, 32)])
def test_indices_bit_exact(N, seed, a, b, blocks, S, R, group):
    api = N.api
    SCR, COL, ROWS, MAP = empty(b + blocks, "i32"), empty(R, "i32"), empty(S * group, "i32"), empty(a, "i32")
    api.sj_pvjp_indices(None, seed, a, b, blocks, S, R, group, SCR.p, COL.p, ROWS.p, MAP.p)
    sync()
    c, r, m = pvjp.indices(seed, a, b, blocks, S, R, group)
    np.testing.assert_array_equal(COL.host(), c)
    np.testing.assert_array_equal(ROWS.host(), r)
    np.testing.assert_array_equal(MAP.host(), m)


def test_cfg5_projection_group(N):
    """A cfg5-sized group (tokens 8192, d 1024, rank 16, 10% of 32-row
    blocks, bf16 donor): basis orthonormality, prepare and coefficients
    against FP64 conditioned on the device Q."""
    n, a, b, donor = 8192, 1024, 512, 1536
    rng = np.random.default_rng(5)
    X = O.round_to(rng.normal(0, 1, (n, a)), "bf16")
    Y = O.round_to(rng.normal(0, 1, (n, donor)), "bf16")
    D = (rng.normal(0, 1, (n, b)) / n).astype(np.float32).astype(np.float64)
    print(f"[pvjp] cfg5-sized n={n} a={a} b={b}", flush=True)
    P = _prepare(N, X, Y, 16, 0.1, 32, 99, ydtype="bf16")
    R, k = P["R"], P["k"]
    assert (R, P["blocks"], P["S"]) == (16, 32, 4)
    q = P["q"]
    assert np.abs(q.T @ q - np.eye(R)).max() < 1e-5
    A_ref, E_ref = pvjp.prepare(X, q, P["rows"], P["blocks"], P["S"])
    assert rel(P["left"], A_ref) < 1e-5 and rel(P["e"], E_ref) < 1e-5
    C = _coefficients(N, P, D)
    assert rel(C.host().reshape(R + k, b), (P["eh"] + P["el"]) @ D) < 1e-5


@pytest.mark.parametrize("n,a,b", [(1024, 256, 640), (8192, 1024, 512)])
def test_row_layout_prepare_and_coefficients_match_transposed(N, n, a, b):
    """sj_pvjp_prepare_rows / sj_pvjp_vjp_rows (X and dY in row layout, as the
    step stores them) give the bits of the transposed-operand entry points."""
    api, lib = N.api, N.load()
    rng = np.random.default_rng(n + a)
    X = O.round_to(rng.normal(0, 1, (n, a)), "bf16")
    Y = O.round_to(rng.normal(0, 1, (n, 2 * b)), "bf16")
    D = (rng.normal(0, 1, (n, b)) / n).astype(np.float32).astype(np.float64)
    P = _prepare(N, X, Y, 16, 0.1, 32, 7, ydtype="bf16")
    R, k, n8 = P["R"], P["k"], P["n8"]
    XR = dev(X, "bf16")
    LEFT, E = empty(a * R), empty((R + k) * n8)
    EH, EL = empty((R + k) * n8, "bf16"), empty((R + k) * n8, "bf16")
    ws = empty(max(lib.sj_pvjp_prepare_workspace_bytes(a, n, R), 256), "u8")
    api.sj_pvjp_prepare_rows(None, XR.p, a, a, n, P["Q"].p, R, P["ROWS"].p, k, cf(P["inverse"]), LEFT.p, E.p, EH.p,
                             EL.p, n8, ws.p, ws.nbytes)
    sync()
    np.testing.assert_array_equal(LEFT.host().reshape(a, R), P["left"])
    np.testing.assert_array_equal(E.host().reshape(R + k, n8), P["e"])
    np.testing.assert_array_equal(EH.host().reshape(R + k, n8), P["eh"])
    np.testing.assert_array_equal(EL.host().reshape(R + k, n8), P["el"])
    C = _coefficients(N, P, D)
    dh, dl = _planes(D)
    DH, DL = dev(dh, "bf16"), dev(dl, "bf16")
    C2 = empty((R + k) * b)
    wsv = empty(max(lib.sj_pvjp_vjp_workspace_bytes(R + k, b, n), 256), "u8")
    api.sj_pvjp_vjp_rows(None, P["EH"].p, P["EL"].p, n8, R + k, n, DH.p, DL.p, b, b, C2.p, b, wsv.p, wsv.nbytes)
    sync()
    np.testing.assert_array_equal(C2.host(), C.host())
