"""Evaluation and cached-inference measurement of the `benchmark` command
(crates/sejong-cli/src/benchmark.rs:71-171) on the native library.

evaluate: bits per byte-token, the mean next-token cross entropy over
`batches` batches of Corpus::batch (seeded with the training seed) divided by
ln 2.  cached_measurement: one held-out sequence, its full-sequence logits,
then a prefill of all but the last `decode` tokens through a fresh KV cache
and teacher-forced decoding of the rest one token at a time (one warm-up
pass, the second pass timed with a synchronisation after each call and the
logits read back after the timed loop), and the largest |cached - full|
over the last token's logits.
"""
from __future__ import annotations

import math
import time

import numpy as np

from .corpus import Corpus
from .model import Model
from .rng import Rng


def evaluate(model: Model, corpus: Corpus, batches: int, seed: int | None = None) -> float:
    """benchmark.rs:71-99."""
    tc = model.tc
    rng = Rng(tc.seed if seed is None else seed)
    total, count = 0.0, 0
    for _ in range(batches):
        ids, tg = corpus.batch(rng, tc.batch, tc.sequence)
        model.set_batch(ids, tg)
        loss = model.forward()
        if not math.isfinite(loss):
            raise ValueError("evaluation produced nonfinite loss")
        total += loss * ids.size
        count += ids.size
    return total / count / math.log(2.0)


def full_logits(model: Model, tokens: np.ndarray) -> np.ndarray:
    """Model::logits of one sequence of the training length: the batch rows
    are independent, so the sequence fills every row of the model's batch
    and the first row's logits are returned [sequence][vocab]."""
    tc = model.tc
    t = np.asarray(tokens, np.int32)
    assert t.size == tc.sequence
    ids = np.tile(t, tc.batch)
    model.set_batch(ids, ids)  # targets do not change the logits
    model.forward()
    return model.logits()[:tc.sequence].copy()


def _distribution(values):
    if not values:
        return None
    o = sorted(values)
    n = len(o)
    return {"samples": n, "mean": sum(values) / n, "median": (o[(n - 1) // 2] + o[n // 2]) / 2,
            "minimum": o[0], "maximum": o[-1]}


def cached_measurement(model: Model, corpus: Corpus, decode: int, seed: int | None = None) -> dict:
    """benchmark.rs:113-171."""
    tc = model.tc
    if not 0 < decode < tc.sequence:
        raise ValueError("decode bytes must be positive and below the sequence")
    ids, _ = corpus.batch(Rng(tc.seed if seed is None else seed), 1, tc.sequence)
    prefix = ids.size - decode
    full = full_logits(model, ids)
    last = None
    prefill_seconds, decode_seconds = 0.0, []
    for pass_ in range(2):
        cache = model.new_cache()
        try:
            model.synchronize()
            t0 = time.perf_counter()
            model.forward_cached(ids[:prefix], cache, read=False)
            model.synchronize()
            if pass_ == 1:
                prefill_seconds = time.perf_counter() - t0
            for token in ids[prefix:]:
                t0 = time.perf_counter()
                model.forward_cached(np.array([token]), cache, read=False)
                model.synchronize()
                if pass_ == 1:
                    decode_seconds.append(time.perf_counter() - t0)
            # the logits are read back after the timed loop (benchmark.rs:150)
            last = cache.logits()
        finally:
            cache.close()
    if not np.all(np.isfinite(last)):
        raise ValueError("cached inference produced nonfinite logits")
    err = float(np.max(np.abs(last.astype(np.float64) - full[-1].astype(np.float64))))
    return {"prefill_tokens": int(prefix), "decode_tokens": int(decode), "prefill_seconds": prefill_seconds,
            "decode_seconds_per_token": _distribution(decode_seconds),
            "decode_tokens_per_second": decode / sum(decode_seconds),
            "cached_vs_full_last_logits_max_abs_error": err,
            "measurement": "same held-out input, one cache warmup, synchronized teacher-forced decoding"}
