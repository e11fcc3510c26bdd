"""NativeValue (native/value.rs:111-160, trained by train_value,
memory.rs:799-1065) on the device against the FP64 oracle, conditioned on
the stored activations: the value logits and loss from the stored SEP rows,
the affine head's gradients, and every body / value-embedding gradient
from the oracle's body backward fed with the head's hidden gradient; then
the AdamW update of the bias (2-D, so it decays) and graph replay."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import rel

pytestmark = pytest.mark.gpu


def _setup(optimizer="adamw"):
    from sejong_amd.model import ModelConfig, TrainConfig
    from sejong_amd.value import NativeValue, ValueMetadata, initial_params
    mc = ModelConfig(width=256, layers=2, heads=4, kv_heads=2, ffn_width=512, context=64, precision="bf16")
    tc = TrainConfig(optimizer=optimizer, batch=8, learning_rate=1e-3, weight_decay=0.1)
    rng = np.random.default_rng(11)
    prompts = [bytes(rng.integers(0, 256, int(rng.integers(3, 40))).astype(np.uint8)) for _ in range(12)]
    meta = ValueMetadata(requests=[f"r{i}" for i in range(12)], prompts=prompts, values=["a", "b", "c", "d", "e"])
    labels = rng.integers(0, 5, 12)
    nv = NativeValue(mc, tc, meta, labels)
    params = initial_params(mc, 5)
    nv.set_params(params)
    return nv, mc, params, labels


def test_value_step_against_oracle():
    from sejong_amd.model import value_layout
    nv, mc, params, labels = _setup()
    try:
        m, T, B, d, n = nv.model, nv.sequence, nv.tc.batch, mc.width, 5
        idx = nv.sample()
        ids, sel = nv.load(idx)
        m.forward_backward()
        loss, _ = m.read_loss()
        grads = m.get_grads().astype(np.float64)
        acts = np.empty(m.activation_count(), np.float32)
        m.export_activations(acts)
        acts = acts.astype(np.float64)
        cfg = dict(d=d, layers=mc.layers, hq=mc.heads, hk=mc.kv, ffn=mc.ffn_width, T=T, B=B, eps=mc.norm_epsilon,
                   theta=mc.rope_theta)
        M = T * B
        A, off = {}, 0
        for name, layer, size in O.acts_layout(cfg):
            if name == "logits":
                size = B * n
            A[(name, layer)] = acts[off:off + size]
            off += size
        P, off = {}, 0
        for name, shape, _ in value_layout(mc, n):
            k = int(np.prod(shape))
            P[name] = (off, shape, params[off:off + k].astype(np.float64).reshape(shape))
            off += k
        hn = A[("hn", -1)].reshape(M, d)
        hs = hn[sel]
        W, b = P["native_value"][2], P["native_bias"][2].ravel()
        logits = hs @ W + b
        dev_logits = A[("logits", -1)].reshape(B, n)
        assert rel(dev_logits, logits) < 1e-5
        lab = labels[np.asarray(idx)]
        lrow, dlog = O.cross_entropy(dev_logits, lab, float(np.float32(1.0) / np.float32(B)))
        assert abs(loss - lrow.mean()) < 1e-6 * abs(loss)
        expect = {"native_value": hs.T @ dlog, "native_bias": dlog.sum(0)[None, :]}
        dh = np.zeros((M, d))
        dh[sel] = dlog @ W.T
        # the body in the oracle's LM layout (embedding / output unused)
        body = [t for t in __import__("sejong_amd.model", fromlist=["layout"]).layout(mc)]
        lm = np.concatenate([P[name][2].ravel() if name in P else np.zeros(int(np.prod(sh)))
                             for name, sh, _ in body])
        gb, demb = O.model_backward_hidden(cfg, lm, acts, dh, dtype="bf16")
        off = 0
        for name, sh, _ in body:
            k = int(np.prod(sh))
            if name in P:
                expect[name] = gb[off:off + k]
            off += k
        expect["native_embedding"] = O.embedding_bwd(demb, ids, 259)
        worst = (None, 0.0)
        for name, (o, shape, _) in P.items():
            k = int(np.prod(shape))
            e = rel(grads[o:o + k], expect[name])
            worst = max(worst, (name, e), key=lambda t: t[1])
            assert e < 1e-3, (name, e)
        print(f"[parity] native value: loss {loss:.7f}; worst grad rel {worst}", flush=True)
    finally:
        nv.close()


def test_value_adamw_steps_graph_and_bias_decay():
    nv, mc, params, _ = _setup()
    ng, _, _, _ = _setup()
    try:
        ng.model.use_graph(True)
        for _ in range(3):
            a, b = nv.train_step(), ng.train_step()
            assert a == b
        np.testing.assert_array_equal(nv.model.get_params(), ng.model.get_params())
        la, lb = nv.model.read_loss()[0], ng.model.read_loss()[0]
        assert la == lb and np.isfinite(la)
    finally:
        nv.close(); ng.close()
