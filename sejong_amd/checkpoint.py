"""Reference-compatible checkpoints of the training step.

A checkpoint is a directory with weights.safetensors (the parameter masters
under their reference names and shapes), optionally optimizer.safetensors
(AdamW: m.<name>, v.<name>, Adam::tensors, crates/sejong-train/src/lib.rs:
239-246; SGD: sgd.version, sgd.sampling_rng, sgd.basis_rng and, with the
parameter VJP, sgd.parameter_rng, control_variate.rs:208-233) and
manifest.json in format 1 (Manifest, crates/sejong-core/src/lib.rs:
548-577): {format, model, step, weights, optimizer, training,
data_fingerprint, rng_state}.  Model::save writes into a staging directory
and renames it (model lib.rs:395-442); the file I/O and the staging run in
libsejong_hip.so (sj_checkpoint_save, sj_safetensors_*).

The reference's half-precision compute dtype is "f16" (DType, core lib.rs:
34-41, has no bf16); this framework's half-precision compute is bf16, so a
bf16 model is recorded as "f16" and a manifest's "f16" loads as bf16.  The
stored tensors are the fp32 masters either way, but the compute dtype
changes across the two frameworks, so both directions emit a
PrecisionMappingWarning unless the caller opts in with half_as_bf16=True.
"""
from __future__ import annotations

import ctypes
import json
import math
import os
import warnings

import numpy as np

from . import _native as N
from .model import HierarchyConfig, Model, ModelConfig, layout

WEIGHTS = "weights.safetensors"
OPTIMIZER = "optimizer.safetensors"
MANIFEST = "manifest.json"
# SgdState::new (control_variate.rs:66-73): the sampling and basis RNGs are
# seeded from the training seed; plain SGD never draws from them
SAMPLING_XOR = 0x38B87C4D9F0A1265
BASIS_XOR = 0xA41239C507EF68BD


def rng_words(state: int) -> np.ndarray:
    """rng_tensor (control_variate.rs:42-47): four 16-bit words as f32."""
    return np.array([(state >> (16 * i)) & 0xFFFF for i in range(4)], np.float32)


def rng_state(words) -> int:
    """read_rng (control_variate.rs:49-63)."""
    w = np.asarray(words, np.float32)
    if w.shape != (4,):
        raise ValueError("RNG state requires four 16-bit words")
    v = 0
    for i, x in enumerate(w):
        if not (math.isfinite(x) and 0 <= x <= 65535 and float(x).is_integer()):
            raise ValueError("invalid optimizer RNG word")
        v |= int(x) << (16 * i)
    return v


class PrecisionMappingWarning(UserWarning):
    """A bf16 model written with the reference's "f16" compute dtype, or an
    "f16" manifest loaded as a bf16 model."""


def _warn_half(what: str, half_as_bf16: bool):
    if not half_as_bf16:
        warnings.warn(PrecisionMappingWarning(
            f"{what}: the reference's half compute dtype f16 is bf16 here (fp32 masters are stored either way); "
            "pass half_as_bf16=True to accept the mapping"), stacklevel=3)


def model_config_json(mc: ModelConfig) -> dict:
    """ModelConfig's serde form (core lib.rs:55-73), fields in declaration
    order; hierarchy / kv_heads only when set."""
    out = {"id": mc.id, "width": mc.width, "layers": mc.layers, "heads": mc.heads, "ffn_width": mc.ffn_width,
           "context": mc.context, "rope_theta": float(np.float32(mc.rope_theta)),
           "norm_epsilon": float(np.float32(mc.norm_epsilon)),
           "precision": "f16" if mc.precision == "bf16" else mc.precision, "seed": mc.seed}
    if mc.hierarchy is not None:
        h = mc.hierarchy
        out["hierarchy"] = {"patch_size": h.patch_size, "encoder_width": h.encoder_width,
                            "encoder_layers": h.encoder_layers, "encoder_heads": h.encoder_heads,
                            "encoder_ffn_width": h.encoder_ffn_width, "decoder_width": h.decoder_width,
                            "decoder_layers": h.decoder_layers, "decoder_heads": h.decoder_heads,
                            "decoder_ffn_width": h.decoder_ffn_width, "local_window": h.local_window,
                            "checkpoint_encoder": False, "checkpoint_decoder": False}
    if mc.kv_heads is not None:
        out["kv_heads"] = mc.kv_heads
    return out


def model_config_from_json(d: dict, half_as_bf16: bool = False) -> ModelConfig:
    known = {"id", "width", "layers", "heads", "ffn_width", "context", "rope_theta", "norm_epsilon", "precision",
             "seed", "hierarchy", "kv_heads", "experts"}
    extra = set(d) - known
    if extra:
        raise ValueError(f"unknown model configuration fields {sorted(extra)}")   # deny_unknown_fields
    if d.get("experts") is not None:
        raise ValueError("mixture-of-experts checkpoints are not loaded by this step driver")
    prec = d.get("precision", "f16")
    if prec == "f16":
        _warn_half("loading an f16 manifest as a bf16 model", half_as_bf16)
    prec = {"f16": "bf16", "f32": "f32"}.get(prec)
    if prec is None:
        raise ValueError(f"precision {d.get('precision')} is not a training compute dtype here")
    h = d.get("hierarchy")
    mc = ModelConfig(width=d.get("width", 512), layers=d.get("layers", 8), heads=d.get("heads", 8),
                     kv_heads=d.get("kv_heads"), ffn_width=d.get("ffn_width", 1536), context=d.get("context", 2048),
                     rope_theta=d.get("rope_theta", 10000.0), norm_epsilon=d.get("norm_epsilon", 1.1920929e-07),
                     precision=prec, seed=d.get("seed", 42), id=d.get("id", "sejong"),
                     hierarchy=None if h is None else HierarchyConfig(
                         **{k: v for k, v in h.items() if k not in ("checkpoint_encoder", "checkpoint_decoder")}))
    if not mc.id:
        raise ValueError("model.id must contain a name")
    mc.validate()
    return mc


def _tensor_lists(named):
    """(count, names, ranks, dims, data pointers, keep-alive) for the C ABI."""
    names, ranks, dims, ptrs, keep = [], [], [], [], []
    for name, arr in named:
        a = np.ascontiguousarray(arr, np.float32)
        keep.append(a)
        names.append(name.encode())
        ranks.append(a.ndim)
        dims.extend(a.shape)
        ptrs.append(a.ctypes.data)
    n = len(names)
    c_names = (ctypes.c_char_p * max(n, 1))(*names)
    c_ranks = (ctypes.c_long * max(n, 1))(*ranks)
    c_dims = (ctypes.c_long * max(len(dims), 1))(*dims)
    c_data = (ctypes.c_void_p * max(n, 1))(*ptrs)
    keep += [c_names, c_ranks, c_dims, c_data]
    return n, c_names, c_ranks, c_dims, c_data, keep


def split(mc: ModelConfig, flat: np.ndarray):
    """[(name, array of the reference shape)] of a reference-layout vector."""
    out, off = [], 0
    for name, shape, _ in layout(mc):
        n = math.prod(shape)
        out.append((name, flat[off:off + n].reshape(shape)))
        off += n
    assert off == flat.size, (off, flat.size)
    return out


def save_arrays(directory: str, mc: ModelConfig, params: np.ndarray, step: int, optimizer: list | None = None,
                training: dict | None = None, data_fingerprint: str | None = None, rng_state: int | None = None,
                half_as_bf16: bool = False):
    """Model::save of host arrays: params in the reference layout; optimizer
    a [(name, array)] list (or None)."""
    if mc.precision == "bf16":
        _warn_half("saving a bf16 model with manifest precision f16", half_as_bf16)
    manifest = {"format": 1, "model": model_config_json(mc), "step": int(step), "weights": WEIGHTS,
                "optimizer": OPTIMIZER if optimizer else None, "training": training,
                "data_fingerprint": data_fingerprint, "rng_state": rng_state}
    w = _tensor_lists(split(mc, np.asarray(params, np.float32)))
    o = _tensor_lists(optimizer or [])
    N.load()
    N.api.sj_checkpoint_save(os.fspath(directory).encode(), json.dumps(manifest, indent=2).encode(),
                             w[0], w[1], w[2], w[3], w[4], o[0] if optimizer else 0, o[1], o[2], o[3], o[4])


def optimizer_tensors(model: Model) -> list:
    """Adam::tensors / SgdState::tensors of a live model."""
    mc, tc = model.mc, model.tc
    if tc.optimizer == "sgd":
        out = [("sgd.version", np.ones(1, np.float32)),
               ("sgd.sampling_rng", rng_words((tc.seed ^ SAMPLING_XOR) & (2 ** 64 - 1))),
               ("sgd.basis_rng", rng_words((tc.seed ^ BASIS_XOR) & (2 ** 64 - 1)))]
        if tc.parameter_vjp is not None:
            out.append(("sgd.parameter_rng", rng_words(model.vjp_info()["rng_state"])))
        return out
    m, v, _ = model.get_adam_state()
    out = []
    for (name, mm), (_, vv) in zip(split(mc, m), split(mc, v)):
        out += [(f"m.{name}", mm), (f"v.{name}", vv)]
    return out


def save(model: Model, directory: str, optimizer: bool = True, training: dict | None = None,
         data_fingerprint: str | None = None, rng_state: int | None = None, half_as_bf16: bool = False,
         corpus=None):
    """Model::save of a live model at its current step (the Adam / SGD step
    count), with its optimizer state unless optimizer=False.  With a corpus,
    the manifest's data_fingerprint is the corpus's fingerprint, as
    save_training writes it (train lib.rs:472-491)."""
    if model.values:
        raise ValueError("checkpoints cover the byte language model (not the NativeValue head)")
    if corpus is not None:
        if data_fingerprint is not None and data_fingerprint != corpus.fingerprint:
            raise ValueError("data_fingerprint differs from the corpus's fingerprint")
        data_fingerprint = corpus.fingerprint
    save_arrays(directory, model.mc, model.get_params(), N.api.sj_model_steps(model.h),
                optimizer_tensors(model) if optimizer else None, training, data_fingerprint, rng_state,
                half_as_bf16=half_as_bf16)


def header(path: str) -> dict:
    N.load()
    n = ctypes.c_size_t()
    N.api.sj_safetensors_header(os.fspath(path).encode(), None, 0, ctypes.byref(n))
    buf = ctypes.create_string_buffer(n.value + 1)
    N.api.sj_safetensors_header(os.fspath(path).encode(), buf, n.value + 1, ctypes.byref(n))
    return json.loads(buf.value.decode())


def read_tensor(path: str, name: str, shape) -> np.ndarray:
    out = np.empty(math.prod(shape), np.float32)
    N.api.sj_safetensors_read(os.fspath(path).encode(), name.encode(), ctypes.c_void_p(out.ctypes.data), out.size)
    return out.reshape(shape)


def load_manifest(directory: str) -> dict:
    """Manifest::load (core lib.rs:559-576)."""
    with open(os.path.join(directory, MANIFEST), "rb") as f:
        m = json.loads(f.read())
    if m.get("format") != 1:
        raise ValueError(f"unsupported artifact format {m.get('format')}")
    for fn in [m["weights"]] + ([m["optimizer"]] if m.get("optimizer") else []):
        if os.path.basename(fn) != fn or fn in ("", ".", ".."):
            raise ValueError("artifact file names must be local basenames")
    return m


def load_arrays(directory: str, half_as_bf16: bool = False):
    """Model::load (model lib.rs:134-170): (ModelConfig, reference-layout
    parameters, manifest, optimizer tensors by name or None)."""
    m = load_manifest(directory)
    mc = model_config_from_json(m["model"], half_as_bf16)
    wpath = os.path.join(directory, m["weights"])
    hdr = {k: v for k, v in header(wpath).items() if k != "__metadata__"}
    expect = layout(mc)
    if len(hdr) != len(expect):
        raise ValueError("model tensor count differs from configuration")
    parts = []
    for name, shape, _ in expect:
        if name not in hdr:
            raise ValueError(f"missing tensor {name}")
        if tuple(hdr[name]["shape"]) != tuple(shape) or hdr[name]["dtype"] != "F32":
            raise ValueError(f"tensor {name} shape or dtype differs from configuration")
        parts.append(read_tensor(wpath, name, shape).ravel())
    params = np.concatenate(parts)
    opt = None
    if m.get("optimizer"):
        opath = os.path.join(directory, m["optimizer"])
        ohdr = {k: v for k, v in header(opath).items() if k != "__metadata__"}
        opt = {k: read_tensor(opath, k, tuple(v["shape"])) for k, v in ohdr.items()}
    return mc, params, m, opt


def check_resume_corpus(manifest: dict, corpus) -> None:
    """The resume check of train_configured (train lib.rs:338-341; the SGD
    driver's control_variate.rs:452): the checkpoint must record this
    corpus's fingerprint."""
    if manifest.get("data_fingerprint") != corpus.fingerprint:
        raise ValueError("resume corpus differs from checkpoint")


def load_into(model: Model, directory: str, half_as_bf16: bool = False, corpus=None) -> dict:
    """Resume a live model from a checkpoint of the same configuration:
    parameters, and the optimizer state (Adam::load_parameters, train
    lib.rs:148-175 with the manifest's step; or the SGD state's parameter
    RNG, control_variate.rs:125-150).  With a corpus, the checkpoint must
    record its fingerprint (check_resume_corpus).  Returns the manifest."""
    mc, params, m, opt = load_arrays(directory, half_as_bf16)
    if layout(mc) != layout(model.mc):
        raise ValueError("checkpoint model configuration differs from the live model")
    if corpus is not None:
        check_resume_corpus(m, corpus)
    model.set_params(params)
    if opt is None:
        return m
    if model.tc.optimizer == "sgd":
        v = opt.get("sgd.version")
        if v is None or v.shape != (1,) or float(v[0]) != 1.0:
            raise ValueError("SGD state version missing or unsupported")
        for key in ("sgd.sampling_rng", "sgd.basis_rng"):
            if key not in opt:
                raise ValueError(f"missing optimizer state {key}")
            rng_state(opt[key])
        if model.tc.parameter_vjp is not None:
            if "sgd.parameter_rng" not in opt:
                raise ValueError("missing optimizer state sgd.parameter_rng")
            model.set_vjp_rng(rng_state(opt["sgd.parameter_rng"]))
        return m
    names = [n for n, _, _ in layout(model.mc)]
    if len(opt) != 2 * len(names):
        raise ValueError("optimizer tensor count mismatch")
    mv = {}
    for p in ("m", "v"):
        parts = []
        for name, shape, _ in layout(model.mc):
            t = opt.get(f"{p}.{name}")
            if t is None:
                raise ValueError(f"missing optimizer tensor {p}.{name}")
            if tuple(t.shape) != tuple(shape):
                raise ValueError("optimizer tensor shape mismatch")
            parts.append(t.ravel())
        mv[p] = np.concatenate(parts)
    model.set_adam_state(mv["m"], mv["v"], int(m["step"]))
    return m
