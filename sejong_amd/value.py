"""Host side of NativeValue: one categorical value read from the SEP row of
a byte request (crates/sejong-model/src/native/value.rs:18-160) and its
training loop (train_value, crates/sejong-train/src/memory.rs:799-1065).

The request packing, the value parameters' initialisation and the request
sampling are host work, as in the reference; the step runs in
libsejong_hip.so (sj_model_create_value / sj_model_set_value_batch).  The
device keeps one padded request length (>= the longest prompt + 2): the pad
bytes after SEP never reach the causal SEP row, so the value logits and
every gradient equal those of the reference's per-batch length.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .model import Model, ModelConfig, TrainConfig, init_params, layout, value_layout
from .rng import Rng

FORMAT = "sejong-native-value-v1"  # value.rs:14
PAD, BOS, SEP = 256, 257, 258      # value.rs:15-16 (pad: the ids' fill value)
VALUE_SEED = 0x76616C7565          # "value": value.rs:59
SAMPLE_SEED = 0x6E6174697665       # "native": memory.rs:929


@dataclass
class ValueMetadata:
    """value.rs:18-27 (the fields the step needs)."""
    requests: list[str]
    prompts: list[bytes]
    values: list[str]
    steps: int = 0
    loss: float = 0.0
    format: str = FORMAT


def pack(prompts: list[bytes], indices, sequence: int) -> tuple[np.ndarray, np.ndarray]:
    """forward_batch's request rows (value.rs:119-137): BOS, the prompt's
    bytes, SEP, then pad; and the SEP position of each row."""
    ids = np.full(len(indices) * sequence, PAD, dtype=np.int32)
    sel = np.zeros(len(indices), dtype=np.int32)
    for row, i in enumerate(indices):
        prompt = prompts[i]
        if len(prompt) + 2 > sequence:
            raise ValueError("native prompt inventory/context mismatch")
        start = row * sequence
        ids[start] = BOS
        ids[start + 1:start + 1 + len(prompt)] = np.frombuffer(bytes(prompt), dtype=np.uint8)
        ids[start + 1 + len(prompt)] = SEP
        sel[row] = start + 1 + len(prompt)
    return ids, sel


def initial_params(mc: ModelConfig, values: int) -> np.ndarray:
    """NativeValue::initialize (value.rs:44-78): the body of
    Model::initialize, then the value embedding [259][d] and head [d][n]
    from Rng(seed ^ "value") normal / sqrt(d), the bias zero; flat in
    NativeValue::parameters order."""
    body = init_params(mc, std=None)
    parts, off = {}, 0
    for name, shape, _ in layout(mc):
        n = math.prod(shape)
        parts[name] = body[off:off + n]
        off += n
    d = mc.width
    rng = Rng(mc.seed ^ VALUE_SEED)
    parts["native_embedding"] = (rng.normal(259 * d) / math.sqrt(d)).astype(np.float32)
    parts["native_value"] = (rng.normal(d * values) / math.sqrt(d)).astype(np.float32)
    parts["native_bias"] = np.zeros(values, np.float32)
    return np.concatenate([parts[name].ravel() for name, _, _ in value_layout(mc, values)]).astype(np.float32)


class NativeValue:
    """A NativeValue model on the GPU: body + value head, trained with the
    configured optimizer (AdamW, or SGD with the optional parameter VJP)."""

    def __init__(self, mc: ModelConfig, tc: TrainConfig, metadata: ValueMetadata, labels, sequence: int | None = None):
        if len(metadata.requests) != len(metadata.prompts) or not metadata.values:
            raise ValueError("native prompt inventory/context mismatch")
        if len(labels) != len(metadata.requests) or not all(0 <= int(i) < len(metadata.values) for i in labels):
            raise ValueError("native value labels invalid")
        longest = max(len(p) for p in metadata.prompts) + 2
        self.sequence = sequence or longest
        if self.sequence < longest or self.sequence > mc.context:
            raise ValueError("native prompt inventory/context mismatch")
        self.mc, self.metadata = mc, metadata
        self.labels = np.asarray(labels, dtype=np.int32)
        self.tc = TrainConfig(**{**tc.__dict__, "sequence": self.sequence})
        self.model = Model(mc, self.tc, values=len(metadata.values))
        self.rng = Rng(mc.seed ^ SAMPLE_SEED)

    def close(self):
        self.model.close()

    def set_params(self, flat: np.ndarray):
        self.model.set_params(flat)

    def sample(self) -> list[int]:
        """train_value's batch draw (memory.rs:939): rng.index(requests) per row."""
        return [self.rng.index(len(self.metadata.requests)) for _ in range(self.tc.batch)]

    def load(self, indices):
        ids, sel = pack(self.metadata.prompts, indices, self.sequence)
        self.model.set_value_batch(ids, sel, self.labels[np.asarray(indices)])
        return ids, sel

    def train_step(self, lr: float | None = None) -> list[int]:
        indices = self.sample()
        self.load(indices)
        self.model.train_step(self.tc.learning_rate if lr is None else lr)
        self.metadata.steps += 1
        return indices
