"""The SGD step driver with the parameter VJP (sj_model_create_sgd; the
cfg5 path: control_variate.rs:503-877 with graph.rs:915-1005) against the
oracle, conditioned on the device's stored activations as in
test_gpu_model.py:

- the step's selection (columns, rows, map) bit-exact against the
  reference generator fed with one next_u64 of Rng::new(seed), the RNG
  carried to the next step;
- the compact gradients (GradientPlan::materialize): for the compressed
  members (q, k, v, gate, up) the factored form left right + tail rows
  built in FP64 from the stored group inputs, the oracle's CGS2 basis of the
  stored donor columns (the up projection of the last layer) and the FP64
  output gradients; dense for the rest; every tensor within 1e-3;
- the update W (1 - lr wd [ndim>1]) - lr clip G with the FP64 norm and the
  clip formed on the device, and the bf16 mirror it writes;
- hipGraph replay equal to eager over two steps; dense SGD (no VJP) equal
  to the AdamW model's gradients; the cfg5 shape's decisions and selection.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from oracle import pvjp as OP
from tests.gpu_util import rel

pytestmark = pytest.mark.gpu

GRAD_TOL = 1e-3


def _cfgs(vjp=True, clip=True, fraction=0.25):
    from sejong_amd.model import ModelConfig, ParameterVjpConfig, TrainConfig
    mc = ModelConfig(width=256, layers=2, heads=4, kv_heads=2, ffn_width=704, context=512, precision="bf16")
    tc = TrainConfig(optimizer="sgd", sequence=512, batch=4, learning_rate=1e-2, weight_decay=0.1,
                     clip_enabled=clip, clip_norm=0.05,
                     parameter_vjp=ParameterVjpConfig(16, fraction, 32, 124) if vjp else None)
    return mc, tc


def _ocfg(mc, tc):
    return dict(d=mc.width, layers=mc.layers, hq=mc.heads, hk=mc.kv, ffn=mc.ffn_width, T=tc.sequence, B=tc.batch,
                eps=mc.norm_epsilon, theta=mc.rope_theta)


def _download(ptr, n, dtype):
    from sejong_amd import _native as N
    out = np.empty(n, dtype)
    N.api.sj_download(ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(ptr), out.nbytes)
    return out


def _model(mc, tc, seed=0):
    from sejong_amd.model import Model, byte_batch, init_params
    from sejong_amd.rng import Rng
    params = init_params(mc, std=0.02, seed=42 + seed)
    ids, tg = byte_batch(Rng(123 + seed), tc.batch, tc.sequence)
    model = Model(mc, tc)
    model.set_params(params)
    model.set_batch(ids, tg)
    return model, params, ids, tg


def _selection(model, mc):
    c = _download(model.buffer("vjp_columns")[0], 16, np.int32)
    r = _download(*model.buffer("vjp_rows"), np.int32) if model.buffer("vjp_rows")[1] else None
    mp = _download(model.buffer("vjp_map")[0], mc.width, np.int32)
    return c, r, mp


def _oracle_selection(mc, tc, draw):
    pv = tc.parameter_vjp
    M = tc.batch * tc.sequence
    R, blocks, S = OP.budget(pv.rank, pv.residual_fraction, pv.block_rows, M, mc.width, mc.ffn_width)
    rng = O.Rng(pv.seed)
    for _ in range(draw):
        seed = rng.next_u64()
    cols, rows, fmap = OP.indices(seed, mc.width, mc.ffn_width, blocks, S, R, pv.block_rows)
    return (R, blocks, S), cols, rows, fmap


def test_vjp_step_gradients_against_oracle():
    _vjp_step_parity(*_cfgs())


def test_vjp_step_gradients_at_cfg5_widths():
    """The same parity at cfg5's widths and depth (12 layers, d 1024, GQA
    16/4, FFN 2752, T 1024, rank 16, residual 0.1 over 32-row blocks, lr
    1e-2, no clip, no weight decay) with the batch cut from 16 sequences to
    1 for the FP64 oracle's time: q|k|v and gate|up still compress at 1024
    tokens (the cost model's decisions at this shape), 60 compressed and 25
    dense matrices."""
    from sejong_amd.model import config
    mc, tc = config("cfg5")
    tc.batch = 1
    print(f"[parity] vjp step at cfg5 widths: d={mc.width} L={mc.layers} F={mc.ffn_width} "
          f"T={tc.sequence} B={tc.batch}", flush=True)
    _vjp_step_parity(mc, tc)


def _vjp_step_parity(mc, tc):
    model, params, ids, tg = _model(mc, tc)
    try:
        L, d, F = mc.layers, mc.width, mc.ffn_width
        info = model.vjp_info()
        assert (info["compressed_matrices"], info["dense_matrices"], info["basis_groups"],
                info["projection_groups"]) == (5 * L, 2 * L + 1, 1, 2 * L)
        model.forward_backward()
        loss, _ = model.read_loss()
        (R, blocks, S), cols, rows, fmap = _oracle_selection(mc, tc, 1)
        dc, dr, dm = _selection(model, mc)
        np.testing.assert_array_equal(dc, cols)
        np.testing.assert_array_equal(dr, rows)
        np.testing.assert_array_equal(dm, fmap)
        r = O.Rng(tc.parameter_vjp.seed); r.next_u64()
        assert model.vjp_info()["rng_state"] == r.state.value
        model.materialize_grads()
        grads = model.get_grads().astype(np.float64)
        cfg = _ocfg(mc, tc)
        acts = np.empty(model.activation_count(), np.float32)
        model.export_activations(acts)
        acts = acts.astype(np.float64)
        A = {}
        off = 0
        for name, layer, size in O.acts_layout(cfg):
            A[(name, layer)] = acts[off:off + size]
            off += size
        lref, gdense, _, dys = O.model_backward(cfg, params.astype(np.float64), acts, ids, tg, "bf16",
                                                want_dys=True)
        assert abs(loss - lref) < 1e-6 * abs(lref)
        M = tc.batch * tc.sequence
        eps = OP.basis_tolerance(M, R)
        Q = OP.basis(A[("u", L - 1)].reshape(M, F), cols, eps)
        expect = gdense.copy()
        pinfo = {name: (rc, o) for name, rc, o in model.param_info()}
        for l in range(L):
            for X, members in ((A[("z", l)].reshape(M, d), ("query", "key", "value")),
                               (A[("z2", l)].reshape(M, d), ("gate", "up"))):
                left, E = OP.prepare(X, Q, rows, blocks, S)
                for mem in members:
                    dy = dys[l][{"query": "q", "key": "k", "value": "v"}.get(mem, mem)]
                    co = E @ dy
                    G = OP.factored_gradient(d, dy.shape[1], [(left, co[:R], co[R:], fmap, 1.0)])
                    (rr, cc), o = pinfo[f"layers.{l}.{mem}"]
                    expect[o:o + rr * cc] = G.ravel()
        worst = (None, 0.0)
        for name, (rr, cc), o in model.param_info():
            e = rel(grads[o:o + rr * cc], expect[o:o + rr * cc])
            if e > worst[1]:
                worst = (name, e)
            assert e < GRAD_TOL, (name, e)
        print(f"[parity] vjp step: loss {loss:.7f} vs {lref:.7f}; worst compact-gradient rel {worst}", flush=True)
    finally:
        model.close()


def test_vjp_sgd_update_and_mirror():
    mc, tc = _cfgs()
    a, params, ids, tg = _model(mc, tc)
    b, _, _, _ = _model(mc, tc)
    try:
        b.forward_backward()          # the same first draw of the parameter RNG as a's step
        b.materialize_grads()
        G = b.get_grads().astype(np.float64)
        a.train_step(tc.learning_rate)
        W1 = a.get_params().astype(np.float64)
        _, norm = a.read_loss()
        ss = float(np.sum(G * G))
        assert abs(norm - np.sqrt(ss)) <= 1e-6 * np.sqrt(ss)
        clip = np.float32(tc.clip_norm / np.sqrt(ss)) if np.sqrt(ss) > tc.clip_norm else np.float32(1.0)
        assert clip < 1.0  # the clip path is exercised
        LR = float(np.float32(np.float32(tc.learning_rate) * clip))
        DECAY = float(np.float32(np.float32(tc.learning_rate) * np.float32(tc.weight_decay)))
        keep = np.ones_like(W1)
        for name, (rr, cc), o in a.param_info():
            if rr > 1:
                keep[o:o + rr * cc] = float(np.float32(1.0 - np.float32(DECAY)))
        exp = params.astype(np.float64) * keep - LR * G
        np.testing.assert_allclose(W1, exp, rtol=2e-6, atol=1e-9)
        # the fused Model::bind cast: mirror = bf16(W) over the internal arena
        pw, n = a.buffer("params")
        pm, _ = a.buffer("mirror")
        w = _download(pw, n, np.float32)
        mbits = _download(pm, n, np.uint16)
        np.testing.assert_array_equal(mbits, (O.round_to(w.astype(np.float64), "bf16").astype(np.float32)
                                              .view(np.uint32) >> 16).astype(np.uint16))
    finally:
        a.close(); b.close()


def test_vjp_graph_replay_two_steps_and_rng():
    mc, tc = _cfgs(fraction=0.1)
    e, _, _, _ = _model(mc, tc)
    g, _, _, _ = _model(mc, tc)
    try:
        g.use_graph(True)
        for _ in range(2):
            e.train_step(); g.train_step()
        np.testing.assert_array_equal(e.get_params(), g.get_params())
        le, lg = e.read_loss()[0], g.read_loss()[0]
        assert le == lg and np.isfinite(le)
        _, cols, rows, fmap = _oracle_selection(mc, tc, 2)
        for m in (e, g):
            c, r, mp = _selection(m, mc)
            np.testing.assert_array_equal(c, cols)
            np.testing.assert_array_equal(r, rows)
            np.testing.assert_array_equal(mp, fmap)
        rng = O.Rng(tc.parameter_vjp.seed); rng.next_u64(); rng.next_u64()
        assert e.vjp_info()["rng_state"] == g.vjp_info()["rng_state"] == rng.state.value
    finally:
        e.close(); g.close()


def test_dense_sgd_matches_adamw_gradients():
    from sejong_amd.model import TrainConfig
    mc, tc = _cfgs(vjp=False, clip=False)
    s, params, ids, tg = _model(mc, tc)
    ta = TrainConfig(sequence=tc.sequence, batch=tc.batch)
    a, _, _, _ = _model(mc, ta)
    try:
        info = s.vjp_info()
        assert (info["compressed_matrices"], info["dense_matrices"], info["basis_groups"]) == (0, 7 * mc.layers + 1, 0)
        s.forward_backward(); a.forward_backward()
        s.materialize_grads()
        G = s.get_grads()
        np.testing.assert_array_equal(G, a.get_grads())
        s.train_step(0.5)
        W1 = s.get_params().astype(np.float64)
        DECAY = float(np.float32(np.float32(0.5) * np.float32(tc.weight_decay)))
        keep = np.ones_like(W1)
        for name, (rr, cc), o in s.param_info():
            if rr > 1:
                keep[o:o + rr * cc] = float(np.float32(1.0 - np.float32(DECAY)))
        np.testing.assert_allclose(W1, params.astype(np.float64) * keep - 0.5 * G.astype(np.float64), rtol=2e-6,
                                   atol=1e-9)
    finally:
        s.close(); a.close()


def test_cfg5_decisions_and_selection():
    """The cfg5 shape (12 layers, d 1024, FFN 2752, 16384 tokens): 60
    compressed and 25 dense matrices, 1 basis and 24 projection groups, and
    the first step's selection equal to the committed golden fixture."""
    import os
    from sejong_amd.model import Model, config
    mc, tc = config("cfg5")
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "pvjp_selection.npz"),
                allow_pickle=False)
    model = Model(mc, tc)
    try:
        info = model.vjp_info()
        assert (info["compressed_matrices"], info["dense_matrices"], info["basis_groups"],
                info["projection_groups"]) == (60, 25, 1, 24)
        rng = np.random.default_rng(7)
        model.set_params(rng.normal(0, 0.02, model.count).astype(np.float32))
        ids = rng.integers(0, 256, tc.batch * tc.sequence).astype(np.int32)
        model.set_batch(ids, np.roll(ids, -1))
        model.train_step()
        loss, _ = model.read_loss()
        assert np.isfinite(loss)
        c, r, mp = _selection(model, mc)
        np.testing.assert_array_equal(c, g["cfg5_columns"])
        np.testing.assert_array_equal(r, g["cfg5_rows"])
        np.testing.assert_array_equal(mp, g["cfg5_map"])
        print(f"[cfg5] first step loss {loss:.5f}", flush=True)
    finally:
        model.close()
