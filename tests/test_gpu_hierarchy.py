"""The hierarchical byte model (cfg3 family: ModelConfig::hierarchy,
architecture.rs:96-137 and 317-393) on the native step driver against the
FP64 oracle (oracle/hierarchy.py).

As for the dense model (test_gpu_model.py), a bf16 end-to-end comparison is
ill-conditioned (near-tie storage roundings flip), so the forward is checked
op by op loosely against the oracle's forward from the same parameters and
the whole backward is recomputed in FP64 from the device's stored
activations: loss and every parameter gradient within 1e-3 relative.  The
fp32 model is compared end to end.  Also: the local window is exercised (96
keys, not a multiple of the 64-key block), graph replay equals eager, and
AdamW covers every tensor (input_projection, which only injected inputs
use, keeps a zero gradient and still decays).
"""
import numpy as np
import pytest

from oracle import hierarchy as H
from oracle import oracle as O
from tests.gpu_util import rel

pytestmark = pytest.mark.gpu

GRAD_TOL = 1e-3


def _configs(precision="bf16", window=96):
    from sejong_amd.model import HierarchyConfig, ModelConfig, TrainConfig
    mc = ModelConfig(width=256, layers=2, heads=4, kv_heads=2, ffn_width=512, context=256, precision=precision,
                     hierarchy=HierarchyConfig(patch_size=4, encoder_width=128, encoder_layers=1, encoder_heads=2,
                                               encoder_ffn_width=256, decoder_width=128, decoder_layers=2,
                                               decoder_heads=2, decoder_ffn_width=384, local_window=window))
    tc = TrainConfig(sequence=256, batch=2, learning_rate=1e-3, weight_decay=0.1)
    return mc, tc


def _ocfg(mc, tc):
    h = mc.hierarchy
    return dict(d=mc.width, layers=mc.layers, hq=mc.heads, hk=mc.kv, ffn=mc.ffn_width, T=tc.sequence, B=tc.batch,
                P=h.patch_size, window=h.local_window, de=h.encoder_width, le=h.encoder_layers, he=h.encoder_heads,
                fe=h.encoder_ffn_width, dd=h.decoder_width, ld=h.decoder_layers, hd=h.decoder_heads,
                fd=h.decoder_ffn_width, eps=mc.norm_epsilon, theta=mc.rope_theta)


def _model(mc, tc, seed=0):
    from sejong_amd.model import Model, byte_batch, init_params
    from sejong_amd.rng import Rng
    params = init_params(mc, std=None, seed=7 + seed)   # Model::initialize scales (global_bos 0)
    params[H._offsets(_ocfg(mc, tc))[0]["global_bos"][0]:][:mc.width] = \
        np.random.default_rng(seed).normal(0, 0.5, mc.width).astype(np.float32)   # a non-zero BOS row
    ids, tg = byte_batch(Rng(31 + seed), tc.batch, tc.sequence)
    model = Model(mc, tc)
    model.set_params(params)
    model.set_batch(ids, tg)
    return model, params, ids, tg


def _per_tensor(model, got, ref):
    out = {}
    for name, (r, c), off in model.param_info():
        n = r * c
        e = ref[off:off + n]
        den = np.linalg.norm(e)
        out[name] = (np.linalg.norm(got[off:off + n] - e) / den) if den > 0 else np.linalg.norm(got[off:off + n])
    return out


def test_hierarchy_layout_matches_oracle():
    from sejong_amd.model import Model
    mc, tc = _configs()
    cfg = _ocfg(mc, tc)
    m = Model(mc, tc)
    try:
        names = [(n, (r, c) if r > 1 or n in ("global_bos",) else (c,)) for n, (r, c), _ in m.param_info()]
        ref = [(n, s) for n, s in H.layout(cfg)]
        assert [n for n, _ in names] == [n for n, _ in ref]
        assert m.count == H.param_count(cfg)
        assert m.activation_count() == sum(n for _, n in H.acts_layout(cfg))
    finally:
        m.close()


@pytest.mark.parametrize("precision", ["bf16", "f32"])
def test_hierarchy_step_against_oracle(precision):
    mc, tc = _configs(precision)
    cfg = _ocfg(mc, tc)
    model, params, ids, tg = _model(mc, tc)
    try:
        print(f"[hierarchy] {precision} forward+backward", flush=True)
        model.forward_backward()
        loss, _ = model.read_loss()
        grads = model.get_grads().astype(np.float64)
        flat = np.empty(model.activation_count(), np.float32)
        model.export_activations(flat)
        dev = H.unpack(cfg, flat.astype(np.float64))
        p64 = params.astype(np.float64)
        if precision == "f32":
            ref_acts = H.model_forward(cfg, p64, ids, "f32")
            for k in ref_acts:
                assert rel(dev[k], ref_acts[k]) < 1e-3, (k, rel(dev[k], ref_acts[k]))
            lref, gref = H.model_backward(cfg, p64, ref_acts, ids, tg, "f32")
            assert abs(loss - lref) <= 1e-4 * abs(lref), (loss, lref)
        else:
            # forward from the same parameters: within a few storage ulps
            ref_acts = H.model_forward(cfg, p64, ids, "bf16")
            for k in ref_acts:
                assert rel(dev[k], ref_acts[k]) < 3e-2, (k, rel(dev[k], ref_acts[k]))
            lref, gref = H.model_backward(cfg, p64, dev, ids, tg, "bf16")
            assert abs(loss - lref) <= 1e-6 * abs(lref), (loss, lref)
        errs = _per_tensor(model, grads, gref)
        worst = max(errs, key=errs.get)
        print(f"[parity] hierarchy {precision}: loss {loss:.6f} vs {lref:.6f}; worst gradient {worst} "
              f"{errs[worst]:.2e}", flush=True)
        for name, e in errs.items():
            assert e < GRAD_TOL, (name, e)
        o, shape = H._offsets(cfg)[0]["input_projection"]
        assert not np.any(grads[o:o + int(np.prod(shape))])
    finally:
        model.close()


def test_hierarchy_graph_replay_and_adamw():
    mc, tc = _configs()
    e, params, ids, tg = _model(mc, tc)
    g, _, _, _ = _model(mc, tc)
    try:
        g.use_graph(True)
        for _ in range(3):
            e.train_step(); g.train_step()
            np.testing.assert_array_equal(e.get_params(), g.get_params())
        assert e.read_loss() == g.read_loss()
        # AdamW touched every tensor, input_projection by weight decay alone
        cfg = _ocfg(mc, tc)
        o, shape = H._offsets(cfg)[0]["input_projection"]
        n = int(np.prod(shape))
        w0, w3 = params[o:o + n].astype(np.float64), e.get_params()[o:o + n].astype(np.float64)
        lr, wd = tc.learning_rate, tc.weight_decay
        decay = float(np.float32(1.0) - np.float32(np.float32(lr) * np.float32(wd)))
        np.testing.assert_allclose(w3, w0 * decay ** 3, rtol=1e-6)
        assert np.isfinite(e.read_loss()[0])
    finally:
        e.close(); g.close()


def test_cfg3_full_configuration_against_oracle():
    """BASELINE cfg3 at its configuration (global d512 x 8 layers, GQA 8/2,
    FFN 1376 over 256 patches of 4 bytes; encoder and decoder d256 x 2,
    4 heads, FFN 768, window 128; T = 1024 bytes; weights N(0, 0.02)) with
    the batch cut from 8 to 2 sequences to bound the FP64 oracle's time:
    the backward recomputed in FP64 from the device's stored activations,
    loss and every gradient within 1e-3 relative; and the loss within 1e-3
    of the oracle's loss from its own bf16 forward (no device values)."""
    from sejong_amd.model import Model, byte_batch, config, init_params
    from sejong_amd.rng import Rng
    mc, tc = config("cfg3")
    tc.batch = 2
    cfg = _ocfg(mc, tc)
    params = init_params(mc, std=0.02, seed=42)
    ids, tg = byte_batch(Rng(123), tc.batch, tc.sequence)
    model = Model(mc, tc)
    try:
        model.set_params(params)
        model.set_batch(ids, tg)
        print("[cfg3] full-configuration forward+backward", flush=True)
        model.forward_backward()
        loss, _ = model.read_loss()
        grads = model.get_grads().astype(np.float64)
        flat = np.empty(model.activation_count(), np.float32)
        model.export_activations(flat)
        dev = H.unpack(cfg, flat.astype(np.float64))
        p64 = params.astype(np.float64)
        print("[cfg3] oracle forward", flush=True)
        ref_acts = H.model_forward(cfg, p64, ids, "bf16")
        for k in ref_acts:
            assert rel(dev[k], ref_acts[k]) < 3e-2, (k, rel(dev[k], ref_acts[k]))
        # the loss gate unconditioned: the oracle's loss from its own forward
        rows, _ = O.cross_entropy(ref_acts["logits"].reshape(-1, O.VOCAB), tg, 1.0)
        lu = float(np.mean(rows))
        print(f"[cfg3] loss {loss:.6f} vs the oracle's own forward {lu:.6f}", flush=True)
        assert abs(loss - lu) <= 1e-3 * abs(lu), (loss, lu)
        print("[cfg3] oracle backward", flush=True)
        lref, gref = H.model_backward(cfg, p64, dev, ids, tg, "bf16")
        assert abs(loss - lref) <= 1e-6 * abs(lref), (loss, lref)
        errs = _per_tensor(model, grads, gref)
        worst = max(errs, key=errs.get)
        print(f"[parity] cfg3 full: loss {loss:.6f} vs {lref:.6f}; worst gradient {worst} {errs[worst]:.2e}",
              flush=True)
        for name, e in errs.items():
            assert e < GRAD_TOL, (name, e)
    finally:
        model.close()
