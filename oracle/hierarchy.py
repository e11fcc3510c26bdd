"""Restatement of the hierarchical model's patch maps (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may import
this module; the product path never does.

The reference kernels (python/sejong_kernels/ops/hierarchy.py:107-172,
launched by crates/sejong-gpu/src/hierarchy_ops.rs:149-278) form their sums
in fp32, one position after another; this restatement does the same in
numpy float32 (elementwise IEEE single operations in the same order), so
the device must match it bit for bit.  Inputs in a bf16 storage dtype are
given as their exact values.

Pinning (tests/test_oracle.py): closed forms (the mean of constant and
linear patches, a partial last patch, patch longer than the sequence, the
shift by one patch with the BOS row first) and the adjoint identities
<pool(x), y> = <x, pool_backward(y)> and <broadcast(x, bos), dy> =
<x, dx> + <bos, dbos>, which fix the backward maps from the forward ones.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


def _store(v, dtype):
    return O.round_to(np.asarray(v, np.float64), dtype) if dtype == "bf16" else np.asarray(v, np.float32).astype(np.float64)


def patch_pool(x, batch, t, patch, dtype="f32"):
    """hierarchy.py:107-119: y[row] = (sum of the patch's rows in order) / count."""
    x = np.asarray(x, np.float32).reshape(batch, t, -1)
    d = x.shape[2]
    patches = -(-t // patch)
    y = np.zeros((batch, patches, d), np.float32)
    for p in range(patches):
        start = p * patch
        count = min(patch, t - start)
        total = np.zeros((batch, d), np.float32)
        for q in range(count):
            total = total + x[:, start + q]
        y[:, p] = total / np.float32(count)
    return _store(y.reshape(batch * patches, d), dtype)


def patch_pool_backward(dy, batch, t, patch):
    """hierarchy.py:122-131: dx[b, pos] = dy[b, pos // patch] / count (fp32)."""
    dy = np.asarray(dy, np.float32)
    d = dy.shape[-1]
    patches = -(-t // patch)
    dy = dy.reshape(batch, patches, d)
    dx = np.zeros((batch, t, d), np.float32)
    for pos in range(t):
        p = pos // patch
        count = min(patch, t - p * patch)
        dx[:, pos] = dy[:, p] / np.float32(count)
    return dx.reshape(batch * t, d).astype(np.float64)


def patch_broadcast(x, bos, batch, t, patch):
    """hierarchy.py:134-143: y[b, pos] = x[b, pos // patch - 1], bos for the first patch."""
    x = np.asarray(x, np.float64)
    d = x.shape[-1]
    patches = -(-t // patch)
    x = x.reshape(batch, patches, d)
    y = np.zeros((batch, t, d))
    for pos in range(t):
        p = pos // patch - 1
        y[:, pos] = x[:, p] if p >= 0 else np.asarray(bos, np.float64).reshape(d)
    return y.reshape(batch * t, d)


def patch_broadcast_backward(dy, batch, t, patch):
    """hierarchy.py:146-172: dx[b, p] = sum over offsets of dy[b, (p+1)*patch
    + offset] (masked positions add 0); dbos = sum over batches, then over the
    first patch's positions; fp32 in that order."""
    dy = np.asarray(dy, np.float32)
    d = dy.shape[-1]
    dy = dy.reshape(batch, t, d)
    patches = -(-t // patch)
    dx = np.zeros((batch, patches, d), np.float32)
    for p in range(patches):
        total = np.zeros((batch, d), np.float32)
        for off in range(patch):
            pos = (p + 1) * patch + off
            total = total + (dy[:, pos] if pos < t else np.float32(0.0))
        dx[:, p] = total
    dbos = np.zeros(d, np.float32)
    for b in range(batch):
        for pos in range(min(patch, t)):
            dbos = dbos + dy[b, pos]
    return dx.reshape(batch * patches, d).astype(np.float64), dbos.astype(np.float64)
