"""The MoE byte Transformer (cfg4 family: ModelConfig::experts, every
block's FFN the MoE branch of Block::apply, architecture.rs:229-242) on the
native step driver against the FP64 oracle (oracle/moe.py model functions).

As for the dense bf16 model, the forward is checked loosely against the
oracle's forward from the same parameters and the whole backward is
recomputed in FP64 from the device's stored activations (router logits,
z2 rows, attention operands): loss and every parameter gradient within
1e-3 relative.  Routing is bit-exact: the device's expert ids and
per-expert counts of every layer equal the reference rule
(softmax, iterative argmax with lowest-index ties, full-softmax weights;
hierarchy.py:175-191, 212-225) applied to the device's stored logits (the fp32 weights within 1e-6).
Graph replay equals eager over three AdamW steps, and every expert's
weights move.
"""
import ctypes

import numpy as np
import pytest

from oracle import moe as OM
from oracle import oracle as O
from tests.gpu_util import rel

pytestmark = pytest.mark.gpu

GRAD_TOL = 1e-3


def _configs(experts=4, top_k=2):
    from sejong_amd.model import ExpertConfig, ModelConfig, TrainConfig
    mc = ModelConfig(width=256, layers=2, heads=4, kv_heads=2, ffn_width=512, context=128, precision="bf16",
                     experts=ExpertConfig(count=experts, top_k=top_k, ffn_width=256))
    tc = TrainConfig(sequence=128, batch=2, learning_rate=1e-3, weight_decay=0.1)
    return mc, tc


def _ocfg(mc, tc):
    return dict(d=mc.width, layers=mc.layers, hq=mc.heads, hk=mc.kv, E=mc.experts.count, K=mc.experts.top_k,
                fe=mc.experts.ffn_width, T=tc.sequence, B=tc.batch, eps=mc.norm_epsilon, theta=mc.rope_theta)


def _model(mc, tc, seed=0):
    from sejong_amd.model import Model, byte_batch, init_params
    from sejong_amd.rng import Rng
    params = init_params(mc, std=None, seed=11 + seed)
    ids, tg = byte_batch(Rng(41 + seed), tc.batch, tc.sequence)
    model = Model(mc, tc)
    model.set_params(params)
    model.set_batch(ids, tg)
    return model, params, ids, tg


def _download(ptr, n, dtype):
    from sejong_amd import _native as N
    out = np.empty(n, dtype)
    N.api.sj_download(ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(ptr), out.nbytes)
    return out


def _check_pack(model, l, M, K, E):
    """The step's pack of layer l (for 8 experts, placed from the top-k
    workgroups' counts) against sj_route_pack on the same routing ids: the
    offsets, the packed slot per position and each slot's position, bit for
    bit."""
    from sejong_amd import _native as N
    ids_ptr, n_ids = model.buffer(f"route_ids.{l}")
    ps_ptr, cap = model.buffer(f"route_pslot.{l}")
    pp_ptr, _ = model.buffer(f"route_ppos.{l}")
    off_ptr, _ = model.buffer(f"route_offsets.{l}")
    bufs = [ctypes.c_void_p() for _ in range(4)]
    for b, nb in zip(bufs, (E * 4, (E + 1) * 4, cap * 4, n_ids * 4)):
        N.api.sj_alloc(nb, ctypes.byref(b))
    try:
        N.api.sj_route_pack(None, ctypes.c_void_p(ids_ptr), M, K, E, None, None, bufs[0], bufs[1], bufs[2], bufs[3],
                            cap)
        N.api.sj_synchronize(None)
        for got, ref, nel in ((off_ptr, bufs[1], E + 1), (ps_ptr, bufs[2], cap), (pp_ptr, bufs[3], n_ids)):
            np.testing.assert_array_equal(_download(got, nel, np.int32), _download(ref.value, nel, np.int32))
    finally:
        for b in bufs:
            N.api.sj_free(b)


def test_moe_model_layout_matches_oracle():
    from sejong_amd.model import Model
    mc, tc = _configs()
    cfg = _ocfg(mc, tc)
    m = Model(mc, tc)
    try:
        names = [n for n, _, _ in m.param_info()]
        assert names == [n for n, _ in OM.layout(cfg)]
        assert m.count == OM.param_count(cfg)
        assert m.activation_count() == sum(n for _, _, n in OM.acts_layout(cfg))
    finally:
        m.close()


def test_moe_model_step_against_oracle():
    mc, tc = _configs()
    cfg = _ocfg(mc, tc)
    M, K, E = tc.batch * tc.sequence, cfg["K"], cfg["E"]
    model, params, ids, tg = _model(mc, tc)
    try:
        print("[moe model] bf16 forward+backward", flush=True)
        model.forward_backward()
        loss, _ = model.read_loss()
        grads = model.get_grads().astype(np.float64)
        flat = np.empty(model.activation_count(), np.float32)
        model.export_activations(flat)
        dev = OM.unpack(cfg, flat)
        p64 = params.astype(np.float64)
        ref_acts = OM.model_forward(cfg, p64, ids, "bf16")
        for k in ref_acts:
            assert rel(dev[k], ref_acts[k]) < 3e-2, (k, rel(dev[k], ref_acts[k]))
        lref, gref, routing = OM.model_backward(cfg, p64, dev, ids, tg, "bf16")
        assert abs(loss - lref) <= 1e-6 * abs(lref), (loss, lref)
        # routing of every layer: bit-exact against the rule on the stored logits
        for l, (rid, rw, counts, _, _) in enumerate(routing):
            _check_pack(model, l, M, K, E)
            d_ids = _download(model.buffer(f"route_ids.{l}")[0], M * K, np.int32).reshape(M, K)
            d_w = _download(model.buffer(f"route_weights.{l}")[0], M * K, np.float32).reshape(M, K)
            d_cnt = _download(model.buffer(f"route_counts.{l}")[0], E, np.int32)
            np.testing.assert_array_equal(d_ids, rid)
            assert rel(d_w, rw) < 1e-6                          # fp32 softmax probabilities
            np.testing.assert_array_equal(d_cnt, counts)
            assert np.all(counts > 0), counts
        worst, errs = 0.0, {}
        for name, (r, c), off in model.param_info():
            e = gref[off:off + r * c]
            errs[name] = np.linalg.norm(grads[off:off + r * c] - e) / max(np.linalg.norm(e), 1e-30)
        worst = max(errs, key=errs.get)
        print(f"[parity] moe model: loss {loss:.6f} vs {lref:.6f}; worst gradient {worst} {errs[worst]:.2e}",
              flush=True)
        for name, e in errs.items():
            assert e < GRAD_TOL, (name, e)
    finally:
        model.close()


def test_moe_model_graph_replay_and_adamw():
    mc, tc = _configs()
    e, params, ids, tg = _model(mc, tc)
    g, _, _, _ = _model(mc, tc)
    try:
        g.use_graph(True)
        for _ in range(3):
            e.train_step(); g.train_step()
            np.testing.assert_array_equal(e.get_params(), g.get_params())
        assert e.read_loss() == g.read_loss()
        assert np.isfinite(e.read_loss()[0])
        w3 = e.get_params()
        for name, (r, c), off in e.param_info():
            if ".experts." in name or name.endswith(".router"):
                assert np.any(w3[off:off + r * c] != params[off:off + r * c]), name
    finally:
        e.close(); g.close()


def test_cfg4_full_configuration_against_oracle():
    """BASELINE cfg4 at its configuration (4 layers, d512, GQA 8/2, every
    FFN 8 SwiGLU experts of 1024 with top-2 routing, T = 512; weights
    N(0, 0.02), router N(0, 1/d) so the logits are N(0, 1)) with the batch
    cut from 8 to 2 sequences for the oracle's time: routing of every layer
    bit-exact against the rule on the stored logits, loss and every
    gradient within 1e-3 of the FP64 backward from the stored activations;
    and the loss within 1e-3 of the oracle's loss from its own bf16
    forward (no device values)."""
    from sejong_amd.model import Model, byte_batch, config, init_params
    from sejong_amd.rng import Rng
    mc, tc = config("cfg4")
    tc.batch = 2
    cfg = _ocfg(mc, tc)
    M, K, E = tc.batch * tc.sequence, cfg["K"], cfg["E"]
    params = init_params(mc, std=0.02, seed=42)
    ids, tg = byte_batch(Rng(123), tc.batch, tc.sequence)
    model = Model(mc, tc)
    try:
        model.set_params(params)
        model.set_batch(ids, tg)
        print("[cfg4] full-configuration forward+backward", flush=True)
        model.forward_backward()
        loss, _ = model.read_loss()
        grads = model.get_grads().astype(np.float64)
        flat = np.empty(model.activation_count(), np.float32)
        model.export_activations(flat)
        dev = OM.unpack(cfg, flat)
        p64 = params.astype(np.float64)
        print("[cfg4] oracle forward", flush=True)
        ref_acts = OM.model_forward(cfg, p64, ids, "bf16")
        for k in ref_acts:
            assert rel(dev[k], ref_acts[k]) < 3e-2, (k, rel(dev[k], ref_acts[k]))
        # the loss gate unconditioned: the oracle's loss from its own forward
        rows, _ = O.cross_entropy(ref_acts[("logits", -1)].reshape(-1, O.VOCAB), tg, 1.0)
        lu = float(np.mean(rows))
        print(f"[cfg4] loss {loss:.6f} vs the oracle's own forward {lu:.6f}", flush=True)
        assert abs(loss - lu) <= 1e-3 * abs(lu), (loss, lu)
        print("[cfg4] oracle backward", flush=True)
        lref, gref, routing = OM.model_backward(cfg, p64, dev, ids, tg, "bf16")
        assert abs(loss - lref) <= 1e-6 * abs(lref), (loss, lref)
        for l, (rid, rw, counts, _, _) in enumerate(routing):
            _check_pack(model, l, M, K, E)
            d_ids = _download(model.buffer(f"route_ids.{l}")[0], M * K, np.int32).reshape(M, K)
            d_w = _download(model.buffer(f"route_weights.{l}")[0], M * K, np.float32).reshape(M, K)
            d_cnt = _download(model.buffer(f"route_counts.{l}")[0], E, np.int32)
            np.testing.assert_array_equal(d_ids, rid)
            assert rel(d_w, rw) < 1e-6
            np.testing.assert_array_equal(d_cnt, counts)
        errs = {}
        for name, (r, c), off in model.param_info():
            e = gref[off:off + r * c]
            errs[name] = np.linalg.norm(grads[off:off + r * c] - e) / max(np.linalg.norm(e), 1e-30)
        worst = max(errs, key=errs.get)
        print(f"[parity] cfg4 full: loss {loss:.6f} vs {lref:.6f}; worst gradient {worst} {errs[worst]:.2e}",
              flush=True)
        for name, e in errs.items():
            assert e < GRAD_TOL, (name, e)
    finally:
        model.close()
