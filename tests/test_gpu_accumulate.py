"""Gradient accumulation of the AdamW step driver (TrainConfig::accumulation;
crates/sejong-train/src/lib.rs:390-415 with Adam::accumulate, :179-198):
`observations` batches per update, each observation's objective seeded with
loss_scale / observations and its loss summary weighted 1 / observations,
the gradients summed in observation order, one norm and one AdamW update."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _setup():
    from sejong_amd.model import config, init_params
    mc, tc = config("cfg2")
    mc.layers, tc.batch, tc.sequence = 2, 2, 128
    return mc, tc, init_params(mc, std=0.02)


def test_accumulated_gradients_loss_and_update():
    """Two observations A, B: the gradient arena after the accumulated
    backward equals fp32(gA / 2 + gB / 2) bit for bit (the seed's halving is
    exact, so every intermediate of each backward is exactly half of the
    single-observation one; the sum is Adam::accumulate's current +
    incoming), the loss is (lossA + lossB) / 2, the step's gradient norm is
    that of the summed gradients, and the update is AdamW's first step on
    them (epsilon 0: every parameter moves by lr * sign(g), after decay)."""
    from sejong_amd.model import Model, byte_batch, layout
    from sejong_amd.rng import Rng
    mc, tc, params = _setup()
    rng = Rng(77)
    ia, ta = byte_batch(rng, tc.batch, tc.sequence)
    ib, tb = byte_batch(rng, tc.batch, tc.sequence)
    model = Model(mc, tc)
    try:
        model.set_params(params)
        model.set_batch(ia, ta); model.forward_backward(); ga = model.get_grads(); la = model.read_loss()[0]
        model.set_batch(ib, tb); model.forward_backward(); gb = model.get_grads(); lb = model.read_loss()[0]
        model.set_batches(np.stack([ia, ib]), np.stack([ta, tb]))
        model.forward_backward()
        gab = model.get_grads()
        lab = model.read_loss()[0]
    finally:
        model.close()
    half = np.float32(0.5)
    want = (ga * half).astype(np.float32) + (gb * half).astype(np.float32)
    np.testing.assert_array_equal(gab, want)
    assert abs(lab - (la + lb) / 2) <= 1e-12 * abs(lab), (lab, la, lb)

    # one training step on the two observations (eager)
    model = Model(mc, tc)
    try:
        model.set_params(params)
        model.set_batches(np.stack([ia, ib]), np.stack([ta, tb]))
        model.use_graph(False)
        model.train_step(tc.learning_rate)
        loss, gnorm = model.read_loss()
        w1 = model.get_params()
        m1, v1, step = model.get_adam_state()
    finally:
        model.close()
    assert step == 1
    assert abs(loss - lab) <= 1e-12 * abs(lab)
    norm = float(np.sqrt(np.sum(gab.astype(np.float64) ** 2)))
    assert abs(gnorm - norm) <= 1e-9 * norm, (gnorm, norm)
    scale = min(1.0, tc.clip_norm / norm) if tc.clip_enabled else 1.0
    np.testing.assert_allclose(m1, (1 - tc.beta1) * gab.astype(np.float64) * scale, rtol=1e-6, atol=1e-30)
    decay = np.concatenate([np.full(int(np.prod(shape)), not is_norm) for _, shape, is_norm in layout(mc)])
    keep = np.where(decay, 1.0 - tc.learning_rate * tc.weight_decay, 1.0)
    want_w = params.astype(np.float64) * keep - tc.learning_rate * np.sign(gab.astype(np.float64))
    err = np.abs(w1 - want_w)
    assert np.all(err <= 1e-6 * tc.learning_rate + 1e-7 * np.abs(want_w)), float(err.max())


def test_accumulated_step_graph_equals_eager_and_set_batch_returns_to_one():
    """Three observations per update: two graph-replayed steps equal two
    eager steps bit for bit (parameters, gradients, moments, losses); then
    set_batch returns to one observation per update and the replayed step
    equals the eager one again."""
    from sejong_amd.model import Model, byte_batch
    from sejong_amd.rng import Rng
    mc, tc, params = _setup()
    rng = Rng(5)
    batches = [byte_batch(rng, tc.batch, tc.sequence) for _ in range(3)]
    ids = np.stack([b[0] for b in batches]); tg = np.stack([b[1] for b in batches])
    out = []
    for graph in (False, True):
        model = Model(mc, tc)
        try:
            model.set_params(params)
            model.set_batches(ids, tg)
            model.use_graph(graph)
            losses = []
            for _ in range(2):
                model.train_step(tc.learning_rate)
                losses.append(model.read_loss())
            model.set_batch(batches[0][0], batches[0][1])
            model.train_step(tc.learning_rate)
            losses.append(model.read_loss())
            m, v, step = model.get_adam_state()
            out.append((model.get_params(), model.get_grads(), m, v, step, losses))
            print(f"[accumulate] graph={graph}: losses {losses}", flush=True)
        finally:
            model.close()
    for name, a, b in zip(("params", "grads", "m", "v"), out[0][:4], out[1][:4]):
        np.testing.assert_array_equal(a, b, err_msg=name)
    assert out[0][4] == out[1][4] == 3
    assert out[0][5] == out[1][5]


def _family(kind):
    from sejong_amd.model import ExpertConfig, HierarchyConfig, ModelConfig, TrainConfig, init_params
    if kind == "moe":
        mc = ModelConfig(width=256, layers=2, heads=4, kv_heads=2, ffn_width=512, context=128, precision="bf16",
                         experts=ExpertConfig(count=4, top_k=2, ffn_width=256))
        tc = TrainConfig(sequence=128, batch=2, learning_rate=1e-3, weight_decay=0.1)
    else:
        mc = ModelConfig(width=256, layers=2, heads=4, kv_heads=2, ffn_width=512, context=256, precision="bf16",
                         hierarchy=HierarchyConfig(patch_size=4, encoder_width=128, encoder_layers=1, encoder_heads=2,
                                                   encoder_ffn_width=256, decoder_width=128, decoder_layers=2,
                                                   decoder_heads=2, decoder_ffn_width=384, local_window=96))
        tc = TrainConfig(sequence=256, batch=2, learning_rate=1e-3, weight_decay=0.1)
    return mc, tc, init_params(mc, std=0.02)


@pytest.mark.parametrize("kind", ["moe", "hier"])
def test_accumulation_across_model_families(kind):
    """The MoE and the hierarchical byte models accumulate the same way as
    the dense one: two observations give fp32(gA / 2 + gB / 2) bit for bit
    (routing, patch pooling and the glue products are linear in the seed,
    which halves exactly) and the loss (lossA + lossB) / 2; two accumulated
    steps replayed from the graph equal two eager ones bit for bit."""
    from sejong_amd.model import Model, byte_batch
    from sejong_amd.rng import Rng
    mc, tc, params = _family(kind)
    rng = Rng(19)
    ia, ta = byte_batch(rng, tc.batch, tc.sequence)
    ib, tb = byte_batch(rng, tc.batch, tc.sequence)
    ids, tg = np.stack([ia, ib]), np.stack([ta, tb])
    model = Model(mc, tc)
    try:
        model.set_params(params)
        model.set_batch(ia, ta); model.forward_backward(); ga = model.get_grads(); la = model.read_loss()[0]
        model.set_batch(ib, tb); model.forward_backward(); gb = model.get_grads(); lb = model.read_loss()[0]
        model.set_batches(ids, tg)
        model.forward_backward()
        gab, lab = model.get_grads(), model.read_loss()[0]
    finally:
        model.close()
    half = np.float32(0.5)
    np.testing.assert_array_equal(gab, (ga * half).astype(np.float32) + (gb * half).astype(np.float32))
    assert abs(lab - (la + lb) / 2) <= 1e-12 * abs(lab), (lab, la, lb)
    out = []
    for graph in (False, True):
        model = Model(mc, tc)
        try:
            model.set_params(params)
            model.set_batches(ids, tg)
            model.use_graph(graph)
            losses = []
            for _ in range(2):
                model.train_step(tc.learning_rate)
                losses.append(model.read_loss())
            out.append((model.get_params(), model.get_grads(), losses))
        finally:
            model.close()
    np.testing.assert_array_equal(out[0][0], out[1][0])
    np.testing.assert_array_equal(out[0][1], out[1][1])
    assert out[0][2] == out[1][2]
    assert np.all(np.isfinite(out[0][0]))


def test_set_batches_rejects_bad_arguments():
    from sejong_amd import _native as N
    from sejong_amd.model import Model, byte_batch
    from sejong_amd.rng import Rng
    mc, tc, params = _setup()
    ia, ta = byte_batch(Rng(1), tc.batch, tc.sequence)
    model = Model(mc, tc)
    try:
        bad = ia.copy(); bad[3] = 300
        with pytest.raises(N.SejongError, match="out of vocabulary"):
            model.set_batches(np.stack([ia, bad]), np.stack([ta, ta]))
        with pytest.raises(N.SejongError, match="observations"):
            model.set_batches(np.tile(ia, 257), np.tile(ta, 257))
    finally:
        model.close()
