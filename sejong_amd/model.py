"""Host side of the byte Transformer step: configuration, reference
parameter layout and initialisation, synthetic byte batches, and a Model /
Adam pair that drives the native step driver (sj_model_* in the C ABI).

Mirrors crates/sejong-core (ModelConfig / TrainConfig defaults, lib.rs:
60-434), crates/sejong-model (layout architecture.rs:63-137, Model::
initialize lib.rs:56-133) and crates/sejong-train (Adam lib.rs:111-247,
Corpus::batch lib.rs:72-88).  All compute runs in libsejong_hip.so.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field

import numpy as np

from . import _native as N
from .rng import Rng

VOCAB = 257  # core lib.rs:305
EOS = 256
F32_EPSILON = float(np.finfo(np.float32).eps)


@dataclass
class HierarchyConfig:
    """crates/sejong-core/src/lib.rs:83-98: byte encoder and decoder around
    the global stack, which runs over patches of patch_size bytes."""
    patch_size: int = 4
    encoder_width: int = 256
    encoder_layers: int = 2
    encoder_heads: int = 4
    encoder_ffn_width: int = 768
    decoder_width: int = 256
    decoder_layers: int = 2
    decoder_heads: int = 4
    decoder_ffn_width: int = 768
    local_window: int = 128


@dataclass
class ExpertConfig:
    """crates/sejong-core/src/lib.rs:100-106: every block's FFN is `count`
    SwiGLU experts of `ffn_width` with top_k routing."""
    count: int = 8
    top_k: int = 2
    ffn_width: int = 1024


@dataclass
class ModelConfig:
    """crates/sejong-core/src/lib.rs:60-111 (dense and hierarchical models;
    no experts on this path)."""
    width: int = 512
    layers: int = 8
    heads: int = 8
    kv_heads: int | None = None
    ffn_width: int = 1536
    context: int = 2048
    rope_theta: float = 10000.0
    norm_epsilon: float = F32_EPSILON
    precision: str = "bf16"  # "f32" | "bf16"
    seed: int = 42
    hierarchy: HierarchyConfig | None = None
    id: str = "sejong"
    experts: ExpertConfig | None = None

    @property
    def kv(self) -> int:
        return self.kv_heads or self.heads

    @property
    def head_dim(self) -> int:
        return self.width // self.heads

    def validate(self):
        if not (self.width > 0 and self.heads > 0 and self.width % self.heads == 0):
            raise ValueError("width must be divisible by heads")
        if self.head_dim % 2:
            raise ValueError("RoPE requires an even head width")
        if not (self.layers > 0 and self.ffn_width > 0 and self.context > 0):
            raise ValueError("layers, ffn_width and context must be positive")
        if self.heads % self.kv:
            raise ValueError("heads must be divisible by kv_heads")
        if self.precision not in ("f32", "bf16"):
            raise ValueError("precision must be f32 or bf16")
        h = self.hierarchy
        if h is not None:  # core lib.rs:163-190
            if not (0 < h.patch_size <= self.context and h.local_window > 0):
                raise ValueError("patch_size must be in 1..=context and local_window must be positive")
            for w, l, hd, f in ((h.encoder_width, h.encoder_layers, h.encoder_heads, h.encoder_ffn_width),
                                (h.decoder_width, h.decoder_layers, h.decoder_heads, h.decoder_ffn_width)):
                if not (w > 0 and l > 0 and hd > 0 and f > 0 and w % hd == 0 and (w // hd) % 2 == 0):
                    raise ValueError("hierarchy stages require positive dimensions and an even head width")


@dataclass
class ParameterVjpConfig:
    """crates/sejong-core/src/lib.rs:447-466."""
    rank: int = 16
    residual_fraction: float = 0.25
    block_rows: int = 32
    seed: int = 124

    def validate(self):
        if not (0 < self.rank <= 2 ** 31 - 1 and 0 < self.block_rows <= 2 ** 31 - 1
                and math.isfinite(self.residual_fraction) and 0.0 < self.residual_fraction <= 1.0):
            raise ValueError("parameter VJP requires positive rank/block_rows and residual_fraction in (0,1]")


@dataclass
class TrainConfig:
    """crates/sejong-core/src/lib.rs:308-362 defaults (AdamW and SGD subset)."""
    optimizer: str = "adamw"  # "adamw" | "sgd"
    parameter_vjp: ParameterVjpConfig | None = None
    sequence: int = 512
    batch: int = 1
    learning_rate: float = 3e-4
    beta1: float = 0.9
    beta2: float = 0.95
    epsilon: float = 0.0
    weight_decay: float = 0.1
    clip_norm: float = 1.0
    clip_enabled: bool = True
    loss_scale: float = 1.0
    seed: int = 123

    def validate(self):
        if self.parameter_vjp is not None:
            if self.optimizer != "sgd":
                raise ValueError("parameter_vjp uses the compact SGD optimizer")
            self.parameter_vjp.validate()
        if self.optimizer not in ("adamw", "sgd"):
            raise ValueError("optimizer must be adamw or sgd")


# BASELINE configurations of this path
def config(name: str) -> tuple[ModelConfig, TrainConfig]:
    if name == "cfg1":  # single pre-norm block, fp32
        return (ModelConfig(width=128, layers=1, heads=4, kv_heads=2, ffn_width=384, context=128,
                            norm_epsilon=1e-6, precision="f32"),
                TrainConfig(sequence=128, batch=2))
    if name == "cfg2":  # 6-layer byte Transformer, bf16, AdamW lr 3e-4 wd 0.01
        return (ModelConfig(width=384, layers=6, heads=6, kv_heads=2, ffn_width=1024, context=512,
                            precision="bf16"),
                TrainConfig(sequence=512, batch=8, learning_rate=3e-4, weight_decay=0.01))
    if name == "cfg5":  # scaled parameter-VJP path: rank 16, 10% residual rows, selected-row SGD lr 1e-2
        # optimizer settings of configs/sejong-parameter-vjp.toml:35-59 (sgd,
        # no clipping, no weight decay, accumulation 1, block_rows 32, seed 124)
        return (ModelConfig(width=1024, layers=12, heads=16, kv_heads=4, ffn_width=2752, context=1024,
                            precision="bf16"),
                TrainConfig(optimizer="sgd", sequence=1024, batch=16, learning_rate=1e-2, weight_decay=0.0,
                            clip_enabled=False,
                            parameter_vjp=ParameterVjpConfig(rank=16, residual_fraction=0.1, block_rows=32,
                                                             seed=124)))
    if name == "cfg3":  # hierarchical byte model; local FFN 3 x width and window 128 (configs/sejong.toml:16-25)
        return (ModelConfig(width=512, layers=8, heads=8, kv_heads=2, ffn_width=1376, context=1024, precision="bf16",
                            hierarchy=HierarchyConfig(patch_size=4, encoder_width=256, encoder_layers=2,
                                                      encoder_heads=4, encoder_ffn_width=768, decoder_width=256,
                                                      decoder_layers=2, decoder_heads=4, decoder_ffn_width=768,
                                                      local_window=128)),
                TrainConfig(sequence=1024, batch=8, learning_rate=3e-4, weight_decay=0.01))
    if name == "cfg4":  # MoE byte Transformer: 8 SwiGLU experts of 1024, top-2 (router logits N(0,1))
        return (ModelConfig(width=512, layers=4, heads=8, kv_heads=2, ffn_width=1024, context=512, precision="bf16",
                            experts=ExpertConfig(count=8, top_k=2, ffn_width=1024)),
                TrainConfig(sequence=512, batch=8, learning_rate=3e-4, weight_decay=0.01))
    raise KeyError(name)


def _stage_layout(prefix: str, d: int, layers: int, heads: int, kv_heads: int, ffn: int,
                  experts: ExpertConfig | None = None):
    """stage_layout (architecture.rs:63-95)."""
    kv = d // heads * kv_heads
    out = []
    for i in range(layers):
        p = f"{prefix}.{i}"
        out += [(f"{p}.attention_norm", (d,), True), (f"{p}.ffn_norm", (d,), True),
                (f"{p}.query", (d, d), False), (f"{p}.key", (d, kv), False), (f"{p}.value", (d, kv), False),
                (f"{p}.attention_output", (d, d), False)]
        if experts is not None:
            fe = experts.ffn_width
            for e in range(experts.count):
                q = f"{p}.experts.{e}"
                out += [(f"{q}.gate", (d, fe), False), (f"{q}.up", (d, fe), False), (f"{q}.down", (fe, d), False)]
            out.append((f"{p}.router", (d, experts.count), False))
        else:
            out += [(f"{p}.gate", (d, ffn), False), (f"{p}.up", (d, ffn), False), (f"{p}.down", (ffn, d), False)]
    return out


def layout(c: ModelConfig) -> list[tuple[str, tuple[int, ...], bool]]:
    """(name, shape, is_norm) in the reference order (architecture.rs:96-137)."""
    d = c.width
    h = c.hierarchy
    glob = _stage_layout("layers", d, c.layers, c.heads, c.kv, c.ffn_width, c.experts)
    if h is None:
        return [("embedding", (VOCAB, d), False)] + glob + [("final_norm", (d,), True), ("output", (d, VOCAB), False)]
    de, dd = h.encoder_width, h.decoder_width
    return ([("embedding", (VOCAB, de), False)]
            + _stage_layout("encoder", de, h.encoder_layers, h.encoder_heads, h.encoder_heads, h.encoder_ffn_width)
            + [("encoder_norm", (de,), True), ("input_projection", (d, de), False),
               ("encoder_to_global", (de, d), False), ("encoder_to_decoder", (de, dd), False),
               ("global_to_decoder", (d, dd), False), ("global_bos", (1, d), False), ("global_norm", (d,), True)]
            + glob
            + _stage_layout("decoder", dd, h.decoder_layers, h.decoder_heads, h.decoder_heads, h.decoder_ffn_width)
            + [("decoder_norm", (dd,), True), ("output_projection", (dd, d), False),
               ("final_norm", (d,), True), ("output", (d, VOCAB), False)])


def value_layout(c: ModelConfig, values: int) -> list[tuple[str, tuple[int, ...], bool]]:
    """NativeValue::parameters order (native/value.rs:89-115): the body
    without embedding and output, then the value embedding (259 rows: bytes,
    pad 256, BOS 257, SEP 258), the value head and its bias."""
    body = [t for t in layout(c) if t[0] not in ("embedding", "output")]
    return body + [("native_embedding", (259, c.width), False), ("native_value", (c.width, values), False),
                   ("native_bias", (1, values), False)]


def param_count(c: ModelConfig) -> int:
    return sum(math.prod(s) for _, s, _ in layout(c))


def init_params(c: ModelConfig, std: float | None = 0.02, seed: int | None = None) -> np.ndarray:
    """Flat fp32 masters in the reference layout.  std=None restates
    Model::initialize (model lib.rs:83-115): N(0, 1/sqrt(fan_in)), /sqrt(2
    depth) for down / attention_output (depth = the layers of the tensor's
    stage), embedding 1/sqrt(d); otherwise every matrix is N(0, std) except
    a router, N(0, 1/sqrt(d)) either way (router logits N(0, 1) on unit-RMS
    rows).  Norm weights are 1, global_bos 0."""
    rng = Rng(c.seed if seed is None else seed)
    h = c.hierarchy
    parts = []
    for name, shape, norm in layout(c):
        n = math.prod(shape)
        if norm:
            parts.append(np.ones(n))
            continue
        if name == "global_bos":
            parts.append(np.zeros(n))
            continue
        if std is None:
            s = 1.0 / math.sqrt(shape[1] if name == "embedding" else shape[0])
            depth = c.layers
            if h is not None and name.startswith("encoder."):
                depth = h.encoder_layers
            elif h is not None and name.startswith("decoder."):
                depth = h.decoder_layers
            if name.endswith(".down") or name.endswith(".attention_output"):
                s /= math.sqrt(2.0 * depth)
        elif name.endswith(".router"):   # cfg4: router logits N(0, 1) over unit-RMS rows
            s = 1.0 / math.sqrt(shape[0])
        else:
            s = std
        parts.append(rng.normal(n, s))
    return np.concatenate(parts).astype(np.float32)


def byte_batch(rng: Rng, batch: int, sequence: int) -> tuple[np.ndarray, np.ndarray]:
    """Synthetic uniform-byte batch: each row is sequence+1 bytes drawn with
    index(256); inputs are [0:T], targets [1:T+1] (the Corpus::batch shift,
    train lib.rs:72-88)."""
    raw = rng.indices(256, batch * (sequence + 1)).reshape(batch, sequence + 1).astype(np.int32)
    return raw[:, :-1].reshape(-1).copy(), raw[:, 1:].reshape(-1).copy()


def _np_ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _padded(v: int) -> int:
    return (v + 7) // 8 * 8


class Cache:
    """Cache (model lib.rs:36-50): the keys and values of one sequence per
    layer on the GPU, its length and capacity."""

    def __init__(self, model: "Model", capacity: int):
        self.model = model
        h = ctypes.c_void_p()
        N.api.sj_cache_create(model.h, capacity, ctypes.byref(h))
        self.h = h
        self.capacity = capacity
        p = ctypes.c_void_p()
        N.api.sj_alloc(4 * _padded(VOCAB), ctypes.byref(p))
        self.dev = p.value

    @property
    def length(self) -> int:
        return N.load().sj_cache_length(self.h)

    def reset(self):
        N.api.sj_cache_reset(self.h)

    def logits(self) -> np.ndarray:
        """The fp32 logits the last forward_cached left (synchronises)."""
        self.model.synchronize()
        out = np.empty(VOCAB, np.float32)
        N.api.sj_download(_np_ptr(out), ctypes.c_void_p(self.dev), out.nbytes)
        return out

    def close(self):
        if self.h:
            N.api.sj_cache_destroy(self.h)
            self.h = None
        if self.dev:
            N.api.sj_free(ctypes.c_void_p(self.dev))
            self.dev = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """One byte Transformer resident on the GPU with its optimizer state
    (AdamW, or SGD with the optional parameter VJP).  values > 0 puts the
    NativeValue head on the body (sejong_amd.value; parameters in
    NativeValue::parameters order, batches through set_value_batch)."""

    def __init__(self, mc: ModelConfig, tc: TrainConfig, stream: int | None = None, values: int = 0):
        mc.validate()
        tc.validate()
        if tc.sequence > mc.context:
            raise ValueError("training requires sequence within context")
        self.mc, self.tc = mc, tc
        cfg = N.ModelConfig(vocab=VOCAB, width=mc.width, layers=mc.layers, heads=mc.heads, kv_heads=mc.kv,
                            ffn_width=mc.ffn_width, sequence=tc.sequence, batch=tc.batch,
                            norm_epsilon=mc.norm_epsilon, rope_theta=mc.rope_theta,
                            precision=N.SJ_BF16 if mc.precision == "bf16" else N.SJ_F32)
        handle = ctypes.c_void_p()
        sgd = adam = None
        if tc.optimizer == "sgd":
            pv = tc.parameter_vjp
            sgd = N.SgdConfig(weight_decay=tc.weight_decay, clip_norm=tc.clip_norm, loss_scale=tc.loss_scale,
                              clip_enabled=int(tc.clip_enabled), vjp_rank=pv.rank if pv else 0,
                              vjp_residual_fraction=pv.residual_fraction if pv else 0.0,
                              vjp_block_rows=pv.block_rows if pv else 0, vjp_seed=pv.seed if pv else 0)
        else:
            adam = N.AdamConfig(beta1=tc.beta1, beta2=tc.beta2, epsilon=tc.epsilon, weight_decay=tc.weight_decay,
                                clip_norm=tc.clip_norm, loss_scale=tc.loss_scale, clip_enabled=int(tc.clip_enabled))
        s = ctypes.c_void_p(stream or 0)
        if mc.experts is not None:
            if values or sgd is not None or mc.hierarchy is not None:
                raise ValueError("the MoE model trains with AdamW on the byte objective")
            ex = N.ExpertConfig(count=mc.experts.count, top_k=mc.experts.top_k, ffn_width=mc.experts.ffn_width)
            N.api.sj_model_create_experts(ctypes.byref(cfg), ctypes.byref(ex), ctypes.byref(adam), s,
                                          ctypes.byref(handle))
        elif mc.hierarchy is not None:
            if values or sgd is not None:
                raise ValueError("the hierarchical model trains with AdamW on the byte objective")
            h = mc.hierarchy
            hc = N.HierarchyConfig(patch_size=h.patch_size, encoder_width=h.encoder_width,
                                   encoder_layers=h.encoder_layers, encoder_heads=h.encoder_heads,
                                   encoder_ffn_width=h.encoder_ffn_width, decoder_width=h.decoder_width,
                                   decoder_layers=h.decoder_layers, decoder_heads=h.decoder_heads,
                                   decoder_ffn_width=h.decoder_ffn_width, local_window=h.local_window)
            N.api.sj_model_create_hierarchy(ctypes.byref(cfg), ctypes.byref(hc), ctypes.byref(adam), s,
                                            ctypes.byref(handle))
        elif values:
            N.api.sj_model_create_value(ctypes.byref(cfg), values, ctypes.byref(adam) if adam else None,
                                        ctypes.byref(sgd) if sgd else None, s, ctypes.byref(handle))
        elif sgd is not None:
            N.api.sj_model_create_sgd(ctypes.byref(cfg), ctypes.byref(sgd), s, ctypes.byref(handle))
        else:
            N.api.sj_model_create(ctypes.byref(cfg), ctypes.byref(adam), s, ctypes.byref(handle))
        self.h = handle
        self.values = values
        self.count = N.load().sj_model_param_count(self.h)
        expect = param_count(mc) if not values else sum(math.prod(sh) for _, sh, _ in value_layout(mc, values))
        assert self.count == expect, (self.count, expect)

    def close(self):
        if self.h:
            N.api.sj_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def param_info(self):
        out = []
        for i in range(N.load().sj_model_param_tensors(self.h)):
            name, r, c, o = ctypes.c_char_p(), ctypes.c_long(), ctypes.c_long(), ctypes.c_long()
            N.api.sj_model_param_info(self.h, i, ctypes.byref(name), ctypes.byref(r), ctypes.byref(c), ctypes.byref(o))
            out.append((name.value.decode(), (r.value, c.value), o.value))
        return out

    def set_params(self, flat: np.ndarray):
        a = np.ascontiguousarray(flat, dtype=np.float32)
        assert a.size == self.count
        N.api.sj_model_set_params(self.h, _np_ptr(a))

    def get_params(self) -> np.ndarray:
        a = np.empty(self.count, np.float32)
        N.api.sj_model_get_params(self.h, _np_ptr(a))
        return a

    def get_grads(self) -> np.ndarray:
        a = np.empty(self.count, np.float32)
        N.api.sj_model_get_grads(self.h, _np_ptr(a))
        return a

    def materialize_grads(self):
        """SGD models: dense + factored gradient of the last backward into the
        gradient arena (GradientPlan::materialize), read with get_grads."""
        N.api.sj_model_materialize_grads(self.h)

    def vjp_info(self) -> dict:
        c, d, b, p, r = ctypes.c_long(), ctypes.c_long(), ctypes.c_long(), ctypes.c_long(), ctypes.c_uint64()
        N.api.sj_model_vjp_info(self.h, ctypes.byref(c), ctypes.byref(d), ctypes.byref(b), ctypes.byref(p),
                                ctypes.byref(r))
        return dict(compressed_matrices=c.value, dense_matrices=d.value, basis_groups=b.value,
                    projection_groups=p.value, rng_state=r.value)

    def set_vjp_rng(self, state: int):
        N.api.sj_model_set_vjp_rng(self.h, ctypes.c_uint64(state))

    def get_adam_state(self):
        m = np.empty(self.count, np.float32); v = np.empty(self.count, np.float32); st = ctypes.c_long()
        N.api.sj_model_get_adam_state(self.h, _np_ptr(m), _np_ptr(v), ctypes.byref(st))
        return m, v, st.value

    def set_adam_state(self, m: np.ndarray, v: np.ndarray, step: int):
        m = np.ascontiguousarray(m, np.float32); v = np.ascontiguousarray(v, np.float32)
        assert m.size == self.count and v.size == self.count
        N.api.sj_model_set_adam_state(self.h, _np_ptr(m), _np_ptr(v), step)

    def steps(self) -> int:
        """Updates applied so far (the checkpoint manifest's step)."""
        return N.api.sj_model_steps(self.h)

    def save(self, directory: str, **kw):
        """Reference-compatible checkpoint (sejong_amd.checkpoint.save)."""
        from . import checkpoint
        checkpoint.save(self, directory, **kw)

    def load(self, directory: str, **kw) -> dict:
        """Resume parameters and optimizer state (sejong_amd.checkpoint.load_into)."""
        from . import checkpoint
        return checkpoint.load_into(self, directory, **kw)

    def set_batch(self, ids: np.ndarray, targets: np.ndarray):
        ids = np.ascontiguousarray(ids, dtype=np.int32); tg = np.ascontiguousarray(targets, dtype=np.int32)
        assert ids.size == self.tc.batch * self.tc.sequence == tg.size
        N.api.sj_model_set_batch(self.h, _np_ptr(ids), _np_ptr(tg), 0)

    def set_batches(self, ids: np.ndarray, targets: np.ndarray):
        """Gradient accumulation (train lib.rs:390-415): ids / targets hold
        `observations` batches ([observations][batch * sequence]); each
        following train_step runs every observation's forward and backward
        (its own batch, seed loss_scale / observations, loss summary weighted
        1 / observations) and one AdamW update on the summed gradients.
        set_batch returns to one observation per update."""
        ids = np.ascontiguousarray(ids, dtype=np.int32); tg = np.ascontiguousarray(targets, dtype=np.int32)
        n = self.tc.batch * self.tc.sequence
        assert ids.size == tg.size and ids.size % n == 0
        N.api.sj_model_set_batches(self.h, _np_ptr(ids), _np_ptr(tg), ids.size // n)

    def set_value_batch(self, ids: np.ndarray, positions: np.ndarray, labels: np.ndarray):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        pos = np.ascontiguousarray(positions, dtype=np.int32); lab = np.ascontiguousarray(labels, dtype=np.int32)
        assert ids.size == self.tc.batch * self.tc.sequence and pos.size == lab.size == self.tc.batch
        N.api.sj_model_set_value_batch(self.h, _np_ptr(ids), _np_ptr(pos), _np_ptr(lab))

    def set_batch_device(self, ids_ptr: int, targets_ptr: int):
        N.api.sj_model_set_batch(self.h, ctypes.c_void_p(ids_ptr), ctypes.c_void_p(targets_ptr), 1)

    def forward_backward(self):
        N.api.sj_model_forward_backward(self.h)

    def use_graph(self, on: bool = True):
        N.api.sj_model_use_graph(self.h, int(on))

    def train_step(self, lr: float | None = None):
        N.api.sj_model_train_step(self.h, ctypes.c_float(self.tc.learning_rate if lr is None else lr))

    def forward(self) -> float:
        """Forward only (Model::logits + cross_entropy) of the staged batch:
        its mean loss, no backward and no update."""
        N.api.sj_model_forward(self.h)
        return self.read_loss()[0]

    def logits(self) -> np.ndarray:
        """fp32 logits [rows][vocab] of the last forward (synchronises)."""
        p, n = self.buffer("logits")
        self.synchronize()
        rows = n // _padded(VOCAB)
        out = np.empty(n, np.float32)
        N.api.sj_download(_np_ptr(out), ctypes.c_void_p(p), out.nbytes)
        return out.reshape(rows, _padded(VOCAB))[:, :VOCAB]

    def new_cache(self, capacity: int | None = None) -> "Cache":
        """Model::new_cache (model lib.rs:359-361): capacity = context."""
        return Cache(self, self.mc.context if capacity is None else capacity)

    def forward_cached(self, tokens, cache: "Cache", read: bool = True) -> np.ndarray | None:
        """Model::forward_cached (model lib.rs:362-372): the fp32 logits of
        the last of `tokens` after running them at the cache's positions.
        read=False only enqueues the call (no synchronisation): the logits
        stay on the device until cache.logits()."""
        t = np.ascontiguousarray(tokens, dtype=np.int32).ravel()
        N.api.sj_model_forward_cached(self.h, cache.h, _np_ptr(t), t.size, ctypes.c_void_p(cache.dev))
        return cache.logits() if read else None

    def read_loss(self) -> tuple[float, float]:
        loss, norm = ctypes.c_double(), ctypes.c_double()
        N.api.sj_model_read_loss(self.h, ctypes.byref(loss), ctypes.byref(norm))
        return loss.value, norm.value

    def activation_count(self) -> int:
        return N.load().sj_model_activation_count(self.h)

    def export_activations(self, out: np.ndarray):
        assert out.dtype == np.float32 and out.size == self.activation_count()
        N.api.sj_model_export_activations(self.h, _np_ptr(out))

    def time_steps(self, steps: int, lr: float | None = None) -> float:
        """Milliseconds for `steps` train steps between two HIP events on the
        model stream (synchronises)."""
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        N.api.sj_event_create(ctypes.byref(a)); N.api.sj_event_create(ctypes.byref(b))
        try:
            s = ctypes.c_void_p(self.stream)
            N.api.sj_event_record(a, s)
            for _ in range(steps):
                self.train_step(lr)
            N.api.sj_event_record(b, s)
            ms = ctypes.c_float()
            N.api.sj_event_elapsed(a, b, ctypes.byref(ms))
            return ms.value
        finally:
            N.api.sj_event_destroy(a); N.api.sj_event_destroy(b)

    def synchronize(self):
        N.api.sj_synchronize(ctypes.c_void_p(self.stream))

    def profile(self, on: bool = True, cold: bool = False, kernels: bool = False, instep: bool = False):
        """Per-op HIP-event timing of eager steps; cold: a 512 MiB buffer is
        written before each op so its operands come from HBM; kernels: each
        GEMM op's kernel is also timed alone ("<op>#kernel" aggregates);
        instep: only those kernel times, with the step's second stream
        running beside (the kernels share the chip as in the step)."""
        N.api.sj_model_profile(self.h, 0 if not on else 4 if instep else 2 if cold else 3 if kernels else 1)

    def profile_collect(self) -> dict[str, tuple[float, int]]:
        """{op name: (total ms, calls)} for the ops run since the last collect
        (a split-K GEMM op also as "<op>#kernel": its GEMM kernel alone);
        profile_kernels then maps each name to the GEMM kernel it launched."""
        n = N.load().sj_model_profile_collect(self.h)
        if n < 0:
            raise N.SejongError(3, "profile collection failed")
        out, self.profile_kernels = {}, {}
        for i in range(n):
            name, ms, calls = ctypes.c_char_p(), ctypes.c_double(), ctypes.c_long()
            kern = ctypes.c_char_p()
            N.api.sj_model_profile_entry(self.h, i, ctypes.byref(name), ctypes.byref(ms), ctypes.byref(calls))
            N.api.sj_model_profile_kernel(self.h, i, ctypes.byref(kern))
            out[name.value.decode()] = (ms.value, calls.value)
            self.profile_kernels[name.value.decode()] = (kern.value or b"").decode()
        return out

    def buffer(self, what: str) -> tuple[int, int]:
        p, n = ctypes.c_void_p(), ctypes.c_long()
        N.api.sj_model_buffer(self.h, what.encode(), ctypes.byref(p), ctypes.byref(n))
        return p.value or 0, n.value

    @property
    def stream(self) -> int:
        return self.buffer("stream")[0]
