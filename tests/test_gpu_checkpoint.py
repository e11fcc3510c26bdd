"""Resume from a reference-compatible checkpoint (sejong_amd.checkpoint):
a model saved after some steps and loaded into a fresh model continues
bit for bit like the uninterrupted run (AdamW moments and step, the SGD
parameter-VJP RNG), for the dense and the hierarchical models."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pair(mc, tc, seed=0):
    from sejong_amd.model import Model, byte_batch, init_params
    from sejong_amd.rng import Rng
    params = init_params(mc, std=0.02, seed=11 + seed)
    ids, tg = byte_batch(Rng(5 + seed), tc.batch, tc.sequence)
    a, b = Model(mc, tc), Model(mc, tc)
    for m in (a, b):
        m.set_params(params)
        m.set_batch(ids, tg)
    return a, b


def test_adamw_resume_is_bit_exact(tmp_path):
    """... with the training corpus's fingerprint in the manifest and the
    resume's corpus check (train lib.rs:338-341, 478-483)."""
    from sejong_amd.corpus import Corpus
    from sejong_amd.model import ModelConfig, TrainConfig
    mc = ModelConfig(width=128, layers=2, heads=2, kv_heads=1, ffn_width=256, context=128, precision="bf16")
    tc = TrainConfig(sequence=128, batch=2, learning_rate=1e-3, weight_decay=0.1)
    (tmp_path / "data").mkdir()
    (tmp_path / "data" / "d.txt").write_bytes(np.random.default_rng(1).integers(0, 256, 4000, np.uint8).tobytes())
    corpus = Corpus.open(tmp_path / "data")
    a, b = _pair(mc, tc)
    try:
        for _ in range(2):
            a.train_step()
        a.save(tmp_path / "ck", rng_state=77, half_as_bf16=True, corpus=corpus)
        man = b.load(tmp_path / "ck", half_as_bf16=True, corpus=corpus)
        assert man["step"] == 2 and man["rng_state"] == 77 and b.steps() == 2
        assert man["data_fingerprint"] == corpus.fingerprint
        ma, va, sa = a.get_adam_state()
        mb, vb, sb = b.get_adam_state()
        np.testing.assert_array_equal(ma, mb); np.testing.assert_array_equal(va, vb); assert sa == sb == 2
        for _ in range(2):
            a.train_step(); b.train_step()
        np.testing.assert_array_equal(a.get_params(), b.get_params())
        assert a.read_loss() == b.read_loss()
    finally:
        a.close(); b.close()


def test_sgd_parameter_vjp_resume(tmp_path):
    from sejong_amd.model import ModelConfig, ParameterVjpConfig, TrainConfig
    mc = ModelConfig(width=256, layers=2, heads=4, kv_heads=2, ffn_width=704, context=512, precision="bf16")
    tc = TrainConfig(optimizer="sgd", sequence=512, batch=4, learning_rate=1e-2, weight_decay=0.0,
                     clip_enabled=False, parameter_vjp=ParameterVjpConfig(16, 0.1, 32, 124))
    a, b = _pair(mc, tc, 1)
    try:
        a.train_step()
        a.save(tmp_path / "ck", half_as_bf16=True)
        b.load(tmp_path / "ck", half_as_bf16=True)
        assert b.vjp_info()["rng_state"] == a.vjp_info()["rng_state"]
        a.train_step(); b.train_step()
        np.testing.assert_array_equal(a.get_params(), b.get_params())
    finally:
        a.close(); b.close()


def test_hierarchy_checkpoint_round_trip(tmp_path):
    from sejong_amd import checkpoint as C
    from sejong_amd.model import HierarchyConfig, ModelConfig, TrainConfig
    mc = ModelConfig(width=256, layers=1, heads=4, kv_heads=2, ffn_width=512, context=256, precision="bf16",
                     hierarchy=HierarchyConfig(patch_size=4, encoder_width=128, encoder_layers=1, encoder_heads=2,
                                               encoder_ffn_width=256, decoder_width=128, decoder_layers=1,
                                               decoder_heads=2, decoder_ffn_width=256, local_window=64))
    tc = TrainConfig(sequence=256, batch=2)
    a, b = _pair(mc, tc, 2)
    try:
        a.train_step()
        a.save(tmp_path / "ck", half_as_bf16=True)
        mc2, params, man, opt = C.load_arrays(tmp_path / "ck", half_as_bf16=True)
        assert mc2.hierarchy == mc.hierarchy and man["model"]["precision"] == "f16"
        b.load(tmp_path / "ck", half_as_bf16=True)
        a.train_step(); b.train_step()
        np.testing.assert_array_equal(a.get_params(), b.get_params())
    finally:
        a.close(); b.close()
