"""The device against the committed golden fixtures (tests/golden/, made by
tests/golden/make_golden.py from the pinned oracle): the cfg1 fp32 step,
the reference's closed-form attention case, routing / pack on fixed logits
and the parameter-VJP selections of the reference check and of cfg5."""
import ctypes
import os

import numpy as np
import pytest

from tests.gpu_util import dev, empty, rel, sync, zeros

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BF, F32 = 4, 0


def _load(name):
    return np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def N():
    from sejong_amd import _native as N
    N.load()
    return N


def test_cfg1_step_against_fixture(N):
    from sejong_amd.model import Model, byte_batch, config, init_params, layout
    from sejong_amd.rng import Rng
    g = _load("cfg1_step")
    mc, tc = config("cfg1")
    model = Model(mc, tc)
    try:
        model.set_params(init_params(mc, std=0.02, seed=42))
        ids, tg = byte_batch(Rng(123), tc.batch, tc.sequence)
        model.set_batch(ids, tg)
        model.forward_backward()
        loss, _ = model.read_loss()
        grads = model.get_grads().astype(np.float64)
    finally:
        model.close()
    assert abs(loss - float(g["loss"])) < 1e-6 * abs(float(g["loss"]))
    off, norms = 0, []
    for name, shape, _ in layout(mc):
        n = int(np.prod(shape))
        norms.append(np.linalg.norm(grads[off:off + n]))
        off += n
    assert rel(np.array(norms), g["grad_norms"]) < 1e-4
    assert rel(grads[g["sample_index"]], g["sample_value"]) < 1e-3


@pytest.mark.parametrize("window", [0, 3])
def test_attention_values_case_against_fixture(N, window):
    """hierarchy_check.rs values() inputs, t 5, 4 query / 2 KV heads, width 4."""
    api = N.api
    g = _load("attention_values")
    t, h, kh, d = 5, 4, 2, 4
    Q, K, V, DY = dev(g["q"]), dev(g["k"]), dev(g["v"]), dev(g["dy"])
    O_, L = empty(t * h * d), empty(t * h)
    api.sj_attention_fwd(None, Q.p, h * d, K.p, kh * d, V.p, kh * d, O_.p, h * d, L.p, F32, 1, t, h, kh, d, window)
    dQ, dK, dV, De = empty(t * h * d), empty(t * kh * d), empty(t * kh * d), empty(t * h)
    api.sj_attention_bwd(None, Q.p, h * d, K.p, kh * d, V.p, kh * d, O_.p, h * d, L.p, DY.p, h * d, dQ.p, h * d, dK.p,
                         kh * d, dV.p, kh * d, De.p, F32, 1, t, h, kh, d, window, None)
    sync()
    for name, buf in (("o", O_), ("lse", L), ("dq", dQ), ("dk", dK), ("dv", dV)):
        assert rel(buf.host(), g[f"{name}_w{window}"]) < 2e-6, name


def test_router_against_fixture(N):
    api = N.api
    g = _load("router")
    logits = g["logits"]
    R, E = logits.shape
    K = g["ids"].shape[1]
    X, IDS, W = dev(logits, "bf16"), empty(R * K, "i32"), empty(R * K)
    api.sj_route_topk(None, X.p, BF, R, E, K, IDS.p, W.p)
    DX = empty(R * E)
    api.sj_route_topk_bwd(None, X.p, BF, IDS.p, W.p, dev(g["dy"]).p, DX.p, R, E, K)
    cap = N.load().sj_route_pack_capacity(R * K, E)
    TOK, SLT = zeros(E * R * K, "i32"), zeros(E * R * K, "i32")
    CNT, OFF, PS, PP = empty(E, "i32"), empty(E + 1, "i32"), empty(cap, "i32"), empty(R * K, "i32")
    api.sj_route_pack(None, IDS.p, R, K, E, TOK.p, SLT.p, CNT.p, OFF.p, PS.p, PP.p, cap)
    sync()
    np.testing.assert_array_equal(IDS.host().reshape(R, K), g["ids"])
    assert rel(W.host(), g["weights"]) < 1e-6
    assert rel(DX.host(), g["dlogits"]) < 1e-5
    counts = CNT.host()
    np.testing.assert_array_equal(counts, g["counts"])
    tok, slt = TOK.host().reshape(E, R * K), SLT.host().reshape(E, R * K)
    for e in range(E):
        np.testing.assert_array_equal(tok[e, :counts[e]], g["tokens"][e, :counts[e]])
        np.testing.assert_array_equal(slt[e, :counts[e]], g["slots"][e, :counts[e]])


@pytest.mark.parametrize("case", ["check", "cfg5"])
def test_pvjp_selection_against_fixture(N, case):
    api = N.api
    g = _load("pvjp_selection")
    if case == "check":
        seed, a, b, blocks, S, R, group = int(g["seed_check"]), 71, 97, 5, 2, 33, 16
    else:
        R, blocks, S = (int(v) for v in g["cfg5_budget"])
        seed, a, b, group = int(g["seed_cfg5"]), 1024, 2752, 32
    SCR, COL, ROWS, MAP = empty(b + blocks, "i32"), empty(R, "i32"), empty(S * group, "i32"), empty(a, "i32")
    api.sj_pvjp_indices(None, seed, a, b, blocks, S, R, group, SCR.p, COL.p, ROWS.p, MAP.p)
    sync()
    np.testing.assert_array_equal(COL.host(), g[f"{case}_columns"])
    np.testing.assert_array_equal(ROWS.host(), g[f"{case}_rows"])
    np.testing.assert_array_equal(MAP.host(), g[f"{case}_map"])
