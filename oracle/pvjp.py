"""Restatement of the parameter-VJP path (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may import
this module; the product path never does.  Integer parts are exact Python
integers; floating-point parts are float64 numpy.

  budget / selects_compression / issued_gemm   parameter_vjp.rs:9-13, 85-130
  indices (SplitMix64 partial Fisher-Yates)    parameter.py:6-62, fed with the
                                               seed parameter_vjp.rs:181-190
  basis (classical Gram-Schmidt twice, drop)   parameter.py:65-128,
                                               tolerance parameter_vjp.rs:214-220
  prepare (A = X^T Q, E rows)                  parameter.py:131-190
  vjp coefficients (E dY)                      parameter_vjp.rs:308-320
  factored gradient / update / norm            parameter.py:193-291,
                                               parameter_vjp.rs:329-530
  graph_statistics (grouping, donor, retain)   graph.rs:551-566, 915-1005

Pinning (tests/test_oracle.py): the reference check program's own index
generator (crates/sejong-gpu/examples/parameter_vjp_check.rs:74-100,
restated as text) on its default shape; the cfg5 budget and compression
decisions; orthonormality and the span of the basis (projector of a QR of
the same columns) and the drop rule on a duplicated column; the factored
gradient equal to X^T D when every block is selected (for any orthonormal
Q); the update and norm closed forms; graph_statistics against the
statistics the reference recorded for its production configuration
(docs/measurements/2026-11-01-architecture-fit/applied.json).
"""
from __future__ import annotations

import math

import numpy as np

from oracle.oracle import Rng

BM, BN, BK = 16, 32, 32
F32_EPS = 2.0 ** -23
F32_MAX = float(np.finfo(np.float32).max)


def issued_gemm(m, n, k):
    """parameter_vjp.rs:9-13."""
    up = lambda v, t: -(-v // t) * t
    return 2 * up(m, BM) * up(n, BN) * up(k, BK)


def budget(rank, residual_fraction, block_rows, n, a, donor):
    """parameter_vjp.rs:85-97 -> (rank, blocks, selected)."""
    r = min(rank, n, a, donor)
    blocks = -(-a // block_rows)
    selected = max(min(math.ceil(blocks * residual_fraction), blocks), 1)
    return r, blocks, selected


def _next_pow2(v):
    return 1 << (v - 1).bit_length() if v > 1 else 1


def selects_compression(rank, residual_fraction, block_rows, n, a, b, donor, uses):
    """parameter_vjp.rs:100-130 (exact integer arithmetic)."""
    if n < a or uses <= 1:
        return False
    r, blocks, selected = budget(rank, residual_fraction, block_rows, n, a, donor)
    if selected == blocks:
        return False
    k = selected * block_rows
    padded = -(-n // BM) * BM
    last = max(r - 1, 0)
    full, tail = last // BN, last % BN
    tri = BN * full * (full + 1) // 2 + tail * (full + 1)
    streaming = 2 * (4 * padded * BN + padded) * tri + 5 * padded * r
    resident = 8 * _next_pow2(n) * _next_pow2(r) * r + 5 * _next_pow2(n) * r
    qr = max(streaming, resident)
    shared = qr + issued_gemm(a, r, n) + issued_gemm(k, n, r)
    own = issued_gemm(r + k, b, n) + issued_gemm(a, b, r)
    return own * uses + shared < issued_gemm(a, b, n) * uses


def _draw(rng: Rng, size: int) -> int:
    """parameter.py:17-22 = Rng::index (rejection below (2^64 - size) mod size)."""
    return rng.index(size)


def indices(seed, A, B, NB, S, R, group):
    """parameter.py:25-62: partial Fisher-Yates over B donor columns (R
    draws) then over NB feature blocks (S draws), one SplitMix64 stream
    started at `seed`.  Returns (columns[R], rows[S*group], map[A])."""
    scratch = list(range(B)) + list(range(NB))
    columns = [0] * R
    rows = [-1] * (S * group)
    fmap = [-1] * A
    rng = Rng(seed)
    for i in range(R):
        j = i + _draw(rng, B - i)
        old, value = scratch[i], scratch[j]
        scratch[i], scratch[j] = value, old
        columns[i] = value
    for i in range(S):
        j = i + _draw(rng, NB - i)
        old, value = scratch[B + i], scratch[B + j]
        scratch[B + i], scratch[B + j] = value, old
        for offset in range(group):
            index, position = value * group + offset, i * group + offset
            rows[position] = index if index < A else -1
            if index < A:
                fmap[index] = position
    return (np.array(columns, np.int32), np.array(rows, np.int32), np.array(fmap, np.int32))


def basis_tolerance(rows, rank):
    """parameter_vjp.rs:214-220: the CGS2 drop threshold, as f32."""
    operations = rows * (4.0 * rank + 1.0)
    roundoff = operations * (F32_EPS / 2.0)
    tol = roundoff / (1.0 - roundoff) if roundoff < 1.0 else math.inf
    return float(np.float32(min(tol, F32_MAX)))


def basis(Y, columns, eps):
    """parameter.py:65-128: Q[:, c] = the selected column c with its
    projection on the previous columns removed twice (classical GS), then
    normalised, or zero if |v|^2 <= eps^2 |original|^2."""
    Y = np.asarray(Y, np.float64)
    n, R = Y.shape[0], len(columns)
    Q = np.zeros((n, R))
    for c in range(R):
        v = Y[:, columns[c]].copy()
        original = v @ v
        for _ in range(2):
            coef = Q[:, :c].T @ v
            v = v - Q[:, :c] @ coef
        mag = v @ v
        Q[:, c] = v / math.sqrt(mag) if mag > eps * eps * original else 0.0
    return Q


def prepare(X, Q, rows, blocks, selected):
    """parameter.py:131-190: A = X^T Q [a][R]; E = [Q^T ; (X[:, row] -
    Q A[row]^T) * blocks/selected for each selected row (zero for -1)]."""
    X = np.asarray(X, np.float64)
    Q = np.asarray(Q, np.float64)
    n, a = X.shape
    R = Q.shape[1]
    A = X.T @ Q
    inverse = float(np.float32(blocks / selected))
    E = np.zeros((R + len(rows), n))
    E[:R] = Q.T
    for i, r in enumerate(rows):
        if r >= 0:
            E[R + i] = (X[:, r] - Q @ A[r]) * inverse
    return A, E


def factored_gradient(m, ncols, terms, dense=None):
    """parameter.py:204-241: G = dense + sum over terms of scale * (left
    right + rows of tail placed by row_map).  term = (left [m][r], right
    [r][n], tail [k][n], row_map [m], scale)."""
    G = np.zeros((m, ncols)) if dense is None else np.array(dense, np.float64, copy=True)
    for left, right, tail, row_map, scale in terms:
        G += scale * (np.asarray(left, np.float64) @ np.asarray(right, np.float64))
        row_map = np.asarray(row_map)
        sel = row_map >= 0
        G[sel] += scale * np.asarray(tail, np.float64)[row_map[sel]]
    return G


def factored_update(W, G, lr, clipping, weight_decay, decays):
    """parameter.py:263-272 with GradientPlan::update's factors
    (parameter_vjp.rs:502-518): W (1 - lr wd [ndim > 1]) - lr clip G."""
    LR = float(np.float32(np.float32(lr) * np.float32(clipping)))
    DECAY = float(np.float32(np.float32(lr) * np.float32(weight_decay)))
    return np.asarray(W, np.float64) * ((1.0 - DECAY) if decays else 1.0) - LR * G


def graph_statistics(matmuls, rank, residual_fraction, block_rows):
    """VjpStatistics of one backward (Graph::propagate's grouping, graph.rs:
    551-566, and compressed_parameter_vjp, graph.rs:915-1005).

    matmuls: the Matmul nodes with a parameter weight, in graph order, as
    (input id, rows n, input width a, output width b).  Nodes whose input has
    n >= a are grouped by input; a group's donor is its widest member (the
    last such member on ties: Rust's max_by_key); the members are retained
    while selects_compression holds for them with the current member count,
    until the set stops shrinking.  A node with n < a, or outside its group's
    retained set, is dense.  A group with retained members is a projection
    group; it creates a basis group when its (n, rank) has none yet."""
    members = {}
    for idx, (inp, n, a, b) in enumerate(matmuls):
        if n >= a:
            members.setdefault(inp, []).append(idx)
    stats = dict(compressed_matrices=0, dense_matrices=0, basis_groups=0, projection_groups=0)
    groups, bases = {}, set()
    for idx in reversed(range(len(matmuls))):  # the backward visits the nodes last first
        inp, n, a, b = matmuls[idx]
        if n < a:
            stats["dense_matrices"] += 1
            continue
        if inp not in groups:
            mem = members[inp]
            donor = mem[0]
            for i in mem:
                if matmuls[i][3] >= matmuls[donor][3]:
                    donor = i
            donor_width = matmuls[donor][3]
            active = set(mem)
            while active:
                count = len(active)
                active = {i for i in active
                          if selects_compression(rank, residual_fraction, block_rows, n, a, matmuls[i][3],
                                                 donor_width, count)}
                if len(active) == count:
                    break
            if active:
                r = budget(rank, residual_fraction, block_rows, n, a, donor_width)[0]
                if (n, r) not in bases:
                    bases.add((n, r))
                    stats["basis_groups"] += 1
                stats["projection_groups"] += 1
            groups[inp] = active
        if idx in groups[inp]:
            stats["compressed_matrices"] += 1
        else:
            stats["dense_matrices"] += 1
    return stats
