"""Checkpoint files (no GPU): the safetensors codec of libsejong_hip.so
against the `safetensors` package of the same version the reference pins in
Cargo.lock (0.8.0; its Python binding wraps the same Rust crate), and
Model::save / Model::load semantics (crates/sejong-model/src/lib.rs:
134-170, 395-538; Manifest, crates/sejong-core/src/lib.rs:548-577) on host
arrays."""
import json
import os

import numpy as np
import pytest

safetensors = pytest.importorskip("safetensors")
import safetensors.numpy as stn  # noqa: E402

from sejong_amd import _native as N  # noqa: E402
from sejong_amd import checkpoint as C  # noqa: E402
from sejong_amd.model import HierarchyConfig, ModelConfig, config, init_params, layout  # noqa: E402


def _write(path, named):
    n, names, ranks, dims, data, keep = C._tensor_lists(named)
    N.load()
    N.api.sj_safetensors_write(str(path).encode(), n, names, ranks, dims, data)


def test_safetensors_version_is_the_reference_pin():
    assert safetensors.__version__ == "0.8.0"


def test_writer_bytes_equal_the_crate(tmp_path):
    rng = np.random.default_rng(0)
    named = [("layers.10.query", rng.normal(size=(3, 5)).astype(np.float32)),
             ("layers.2.query", rng.normal(size=(5, 2)).astype(np.float32)),
             ("final_norm", np.ones(7, np.float32)), ("global_bos", np.zeros((1, 4), np.float32)),
             ("m.embedding", rng.normal(size=(2, 3)).astype(np.float32)), ("sgd.version", np.ones(1, np.float32)),
             ("empty", np.zeros((0, 3), np.float32)), ("ünï\"q", np.arange(3, dtype=np.float32))]
    _write(tmp_path / "a.safetensors", named)
    ref = stn.save(dict(named))
    assert (tmp_path / "a.safetensors").read_bytes() == ref
    # and the crate reads it back
    back = stn.load_file(str(tmp_path / "a.safetensors"))
    for k, v in named:
        np.testing.assert_array_equal(back[k], v)


def test_reader_and_header_checks(tmp_path):
    rng = np.random.default_rng(1)
    a = rng.normal(size=(4, 3)).astype(np.float32)
    p = tmp_path / "w.safetensors"
    stn.save_file({"x": a, "y": np.arange(5, dtype=np.float32)}, str(p))
    h = C.header(p)
    assert h["x"]["shape"] == [4, 3] and h["x"]["dtype"] == "F32"
    np.testing.assert_array_equal(C.read_tensor(p, "x", (4, 3)), a)
    with pytest.raises(N.SejongError, match="missing tensor z"):
        C.read_tensor(p, "z", (1,))
    with pytest.raises(N.SejongError, match="shape or dtype differs"):
        C.read_tensor(p, "x", (5, 3))
    q = tmp_path / "bad.safetensors"
    stn.save_file({"x": np.array([1.0, np.nan], np.float32)}, str(q))
    with pytest.raises(N.SejongError, match="nonfinite"):
        C.read_tensor(q, "x", (2,))
    r = tmp_path / "f64.safetensors"
    stn.save_file({"x": np.ones(2)}, str(r))
    with pytest.raises(N.SejongError, match="shape or dtype differs"):
        C.read_tensor(r, "x", (2,))
    t = tmp_path / "trunc.safetensors"
    t.write_bytes(p.read_bytes()[:-8])
    with pytest.raises(N.SejongError, match="invalid data offsets"):
        C.header(t)


def _small_cfgs():
    dense = ModelConfig(width=32, layers=2, heads=4, kv_heads=2, ffn_width=48, context=64, precision="bf16")
    hier = ModelConfig(width=32, layers=1, heads=4, kv_heads=2, ffn_width=48, context=64, precision="f32",
                       hierarchy=HierarchyConfig(patch_size=4, encoder_width=16, encoder_layers=1, encoder_heads=2,
                                                 encoder_ffn_width=24, decoder_width=16, decoder_layers=1,
                                                 decoder_heads=2, decoder_ffn_width=24, local_window=8))
    return dense, hier


@pytest.mark.parametrize("which", [0, 1])
def test_save_load_round_trip_and_manifest(tmp_path, which):
    mc = _small_cfgs()[which]
    params = init_params(mc, std=None, seed=3)
    rng = np.random.default_rng(2)
    opt = []
    for name, shape, _ in layout(mc):
        opt += [(f"m.{name}", rng.normal(size=shape).astype(np.float32)),
                (f"v.{name}", rng.random(size=shape).astype(np.float32))]
    d = tmp_path / "run" / "step-00000007"
    C.save_arrays(d, mc, params, 7, opt, training=None, data_fingerprint="abc", rng_state=12345,
                  half_as_bf16=True)
    assert sorted(os.listdir(d)) == ["manifest.json", "optimizer.safetensors", "weights.safetensors"]
    assert [f for f in os.listdir(d.parent) if f.startswith(".")] == []      # no staging left behind
    m = json.loads((d / "manifest.json").read_text())
    assert list(m) == ["format", "model", "step", "weights", "optimizer", "training", "data_fingerprint",
                       "rng_state"]
    assert m["format"] == 1 and m["step"] == 7 and m["rng_state"] == 12345
    assert m["model"]["precision"] == ("f16" if mc.precision == "bf16" else "f32")
    assert list(m["model"])[:10] == ["id", "width", "layers", "heads", "ffn_width", "context", "rope_theta",
                                     "norm_epsilon", "precision", "seed"]
    assert np.float32(m["model"]["norm_epsilon"]) == np.float32(mc.norm_epsilon)
    # the weights file is exactly what the reference's save_tensors writes
    ref = stn.save({name: arr for name, arr in C.split(mc, params)})
    assert (d / "weights.safetensors").read_bytes() == ref
    mc2, p2, m2, o2 = C.load_arrays(d, half_as_bf16=True)
    assert layout(mc2) == layout(mc) and mc2.precision == mc.precision and mc2.hierarchy == mc.hierarchy
    np.testing.assert_array_equal(p2, params)
    for k, v in opt:
        np.testing.assert_array_equal(o2[k], v)
    # Model::save refuses an existing destination
    with pytest.raises(N.SejongError, match="already exists"):
        C.save_arrays(d, mc, params, 8, half_as_bf16=True)


def test_load_rejects_mismatches(tmp_path):
    mc, _ = _small_cfgs()
    params = init_params(mc, std=0.02)
    d = tmp_path / "ck"
    C.save_arrays(d, mc, params, 1, half_as_bf16=True)
    m = json.loads((d / "manifest.json").read_text())
    # a tensor missing from the weights file
    named = [(n, a) for n, a in C.split(mc, params) if n != "final_norm"]
    os.remove(d / "weights.safetensors")
    _write(d / "weights.safetensors", named)
    with pytest.raises(ValueError, match="tensor count differs"):
        C.load_arrays(d, half_as_bf16=True)
    named.append(("final_norm", np.ones(33, np.float32)))
    os.remove(d / "weights.safetensors")
    _write(d / "weights.safetensors", named)
    with pytest.raises(ValueError, match="final_norm shape or dtype differs"):
        C.load_arrays(d, half_as_bf16=True)
    m["format"] = 2
    (d / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(ValueError, match="unsupported artifact format 2"):
        C.load_arrays(d, half_as_bf16=True)
    m["format"] = 1
    m["weights"] = "../w.safetensors"
    (d / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(ValueError, match="local basenames"):
        C.load_arrays(d, half_as_bf16=True)
    m["weights"] = "weights.safetensors"
    m["model"]["unknown"] = 1
    (d / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(ValueError, match="unknown model configuration"):
        C.load_arrays(d, half_as_bf16=True)


def test_rng_words_round_trip():
    for s in (0, 1, 124, 0xFFFFFFFFFFFFFFFF, 0x38B87C4D9F0A1265 ^ 123):
        w = C.rng_words(s)
        assert w.dtype == np.float32 and w.shape == (4,)
        assert C.rng_state(w) == s
    with pytest.raises(ValueError):
        C.rng_state(np.array([1.5, 0, 0, 0], np.float32))


def test_cfg2_manifest_model_fields():
    mc, _ = config("cfg2")
    j = C.model_config_json(mc)
    assert j["precision"] == "f16" and j["kv_heads"] == 2 and "hierarchy" not in j
    mc3, _ = config("cfg3")
    j3 = C.model_config_json(mc3)
    assert j3["hierarchy"]["local_window"] == 128 and j3["hierarchy"]["checkpoint_encoder"] is False
    back = C.model_config_from_json(j3, half_as_bf16=True)
    assert layout(back) == layout(mc3)


def test_half_precision_mapping_is_reported(tmp_path):
    """A bf16 model is written with the reference's f16 compute dtype and an
    f16 manifest loads as bf16: both directions warn unless the caller opts
    in; an f32 model round-trips silently."""
    import warnings
    mc, _ = _small_cfgs()
    assert mc.precision == "bf16"
    params = init_params(mc, std=0.02)
    with pytest.warns(C.PrecisionMappingWarning, match="manifest precision f16"):
        C.save_arrays(tmp_path / "a", mc, params, 1)
    with pytest.warns(C.PrecisionMappingWarning, match="f16 manifest as a bf16"):
        mc2, _, _, _ = C.load_arrays(tmp_path / "a")
    assert mc2.precision == "bf16"
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        C.load_arrays(tmp_path / "a", half_as_bf16=True)
        mc.precision = "f32"
        C.save_arrays(tmp_path / "b", mc, params, 1)
        assert C.load_arrays(tmp_path / "b")[0].precision == "f32"


def test_data_fingerprint_written_and_checked_on_resume(tmp_path):
    """save_training writes the corpus fingerprint as data_fingerprint
    (train lib.rs:472-491) and a resume refuses a checkpoint of another
    corpus (lib.rs:338-341): the manifest carries Corpus.fingerprint, the
    same corpus passes check_resume_corpus and a different one fails."""
    from sejong_amd.corpus import Corpus
    rng = np.random.default_rng(5)
    (tmp_path / "a").mkdir()
    (tmp_path / "a" / "x.txt").write_bytes(rng.integers(0, 256, 3000, dtype=np.uint8).tobytes())
    (tmp_path / "b").mkdir()
    (tmp_path / "b" / "x.txt").write_bytes(rng.integers(0, 256, 3000, dtype=np.uint8).tobytes())
    ca, cb = Corpus.open(tmp_path / "a"), Corpus.open(tmp_path / "b")
    assert ca.fingerprint != cb.fingerprint and len(ca.fingerprint) == 64
    mc, _ = _small_cfgs()
    d = tmp_path / "ck"
    C.save_arrays(d, mc, init_params(mc, std=0.02), 3, data_fingerprint=ca.fingerprint)
    m = C.load_manifest(d)
    assert m["data_fingerprint"] == ca.fingerprint
    C.check_resume_corpus(m, ca)
    with pytest.raises(ValueError, match="resume corpus differs from checkpoint"):
        C.check_resume_corpus(m, cb)
