"""Pins the FP64 oracle before anything is checked against it.

Each test checks one oracle function against something that does not share
its code: published test vectors, the reference's own check programs
(restated from their text), closed forms, invariants, finite differences and
brute force.  A plausible slip in the oracle (dropped term, wrong sign or
index, transposed operand) fails at least one of them.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def values(n, offset):
    """Closed-form inputs of crates/sejong-gpu/examples/hierarchy_check.rs:11-15."""
    return np.array([((i * 17 + offset) % 41 - 20.0) / 31.0 for i in range(n)], dtype=np.float32).astype(np.float64)


# ------------------------------------------------------------------ RNG
def test_splitmix64_published_vectors():
    # SplitMix64 reference outputs (Vigna's splitmix64.c / Java SplittableRandom).
    r = O.Rng(1234567)
    assert [r.next_u64() for _ in range(5)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]
    assert O.Rng(0).next_u64() == 0xE220A8397B1DCDAF


def test_rng_index_rejection_threshold():
    # index(n) rejects draws below (2^64 - n) mod n (core lib.rs:610-619);
    # for powers of two the threshold is 0 so index == next_u64 % n.
    a, b = O.Rng(7), O.Rng(7)
    for _ in range(100):
        assert a.index(256) == b.next_u64() % 256
    # n = 3: threshold = 2^64 mod 3 = 1; brute-force the accept rule
    a, b = O.Rng(11), O.Rng(11)
    thr = (2 ** 64) % 3
    for _ in range(50):
        got = a.index(3)
        while True:
            x = b.next_u64()
            if x >= thr:
                break
        assert got == x % 3


def test_rng_uniform_and_normal_moments():
    r = O.Rng(42)
    u = np.array([r.uniform() for _ in range(20000)])
    assert 0 < u.min() and u.max() < 1 and abs(u.mean() - 0.5) < 0.01
    z = O.Rng(42).normal_fill(200000, 0.02)
    assert abs(z.mean()) < 2e-4 and abs(z.std() - 0.02) < 2e-4


# ------------------------------------------------------------ rounding
def _bf16_bits(x32):
    b = x32.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def test_round_bf16_matches_bit_trick():
    rng = np.random.default_rng(0)
    x = rng.normal(0, 1, 100000).astype(np.float32) * np.float32(2.0) ** rng.integers(-60, 60, 100000).astype(np.float32)
    # exact ties: low 16 bits == 0x8000 (odd and even upper halves)
    ties = (rng.integers(0, 2 ** 31, 1000).astype(np.uint32) & 0xFFFF0000 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, np.array([1e-40, -3e-39, 0.0], np.float32)])
    np.testing.assert_array_equal(O.round_to(x.astype(np.float64), "bf16"), _bf16_bits(x))


def test_round_f32():
    x = np.random.default_rng(1).normal(size=1000)
    np.testing.assert_array_equal(O.round_to(x, "f32"), x.astype(np.float32).astype(np.float64))


# --------------------------------------------------------------- matmul
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul_vs_numpy(ta, tb):
    rng = np.random.default_rng(2)
    M, N, K = 13, 7, 29
    A = rng.normal(size=(K, M) if ta else (M, K))
    B = rng.normal(size=(N, K) if tb else (K, N))
    ref = (A.T if ta else A) @ (B.T if tb else B)
    np.testing.assert_allclose(O.matmul(A, B, ta, tb), ref, rtol=1e-12, atol=1e-12)


# -------------------------------------------------------------- RMSNorm
def test_rmsnorm_closed_form_and_scale_invariance():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(5, 16)); w = rng.normal(size=16)
    y = O.rmsnorm_fwd(x, w, 0.0)
    np.testing.assert_allclose(y, O.rmsnorm_fwd(7.5 * x, w, 0.0), rtol=1e-13)
    # unit weights: every row has unit RMS
    np.testing.assert_allclose(np.sqrt((O.rmsnorm_fwd(x, np.ones(16), 0.0) ** 2).mean(1)), 1.0, rtol=1e-13)


def _fd_vjp(f, x, dy, eps=1e-6, ndir=3, seed=0):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(ndir):
        e = rng.normal(size=x.shape)
        out.append((e, ((f(x + eps * e) - f(x - eps * e)) * dy).sum() / (2 * eps)))
    return out


def test_rmsnorm_backward_finite_difference():
    rng = np.random.default_rng(4)
    R, D, eps = 6, 24, 1e-6
    x = rng.normal(size=(R, D)); w = rng.normal(size=D); dy = rng.normal(size=(R, D))
    acc = rng.normal(size=(R, D))
    dx, dw = O.rmsnorm_bwd(x, w, dy, eps, dx_acc=acc)
    for e, fd in _fd_vjp(lambda xx: O.rmsnorm_fwd(xx, w, eps), x, dy):
        assert abs(((dx - acc) * e).sum() - fd) < 1e-7 * max(1, abs(fd))
    for e, fd in _fd_vjp(lambda ww: O.rmsnorm_fwd(x, ww, eps), w, dy):
        assert abs((dw * e).sum() - fd) < 1e-7 * max(1, abs(fd))
    # eps = 0: y is scale invariant in x, so sum(dx * x) = 0 per row
    dx0, _ = O.rmsnorm_bwd(x, w, dy, 0.0)
    np.testing.assert_allclose((dx0 * x).sum(1), 0.0, atol=1e-12)


# ----------------------------------------------------------------- RoPE
def test_rope_closed_form_inverse_and_norm():
    rng = np.random.default_rng(5)
    T, H, D = 7, 3, 8
    x = rng.normal(size=(2 * T, H * D))
    y = O.rope(x, T, H, D)
    # position 0 is the identity
    np.testing.assert_allclose(y[0], x[0], rtol=0, atol=0)
    # position 1, pair 0: angle = 1 rad
    a, b = x[1, 0], x[1, 1]
    np.testing.assert_allclose(y[1, :2], [a * math.cos(1) - b * math.sin(1), a * math.sin(1) + b * math.cos(1)], rtol=1e-14)
    # position 3, pair 2: angle = 3 * 10000^(-4/8)
    ang = 3 * 10000.0 ** (-4 / 8)
    a, b = x[3, D + 4], x[3, D + 5]
    np.testing.assert_allclose(y[3, D + 4:D + 6], [a * math.cos(ang) - b * math.sin(ang), a * math.sin(ang) + b * math.cos(ang)], rtol=1e-13)
    # rotation: pair norms preserved, inverse undoes
    np.testing.assert_allclose((y.reshape(-1, 2) ** 2).sum(1), (x.reshape(-1, 2) ** 2).sum(1), rtol=1e-13)
    np.testing.assert_allclose(O.rope(y, T, H, D, inverse=True), x, atol=1e-13)
    # second batch row-block restarts positions (pos = row mod T)
    np.testing.assert_allclose(y[T], x[T])


# ------------------------------------------------------------ Attention
def _attention_reference_check(q, k, v, dy, t, h, kh, d, window):
    """Text restatement of attention_reference, gpu/examples/hierarchy_check.rs:16-77."""
    out = np.zeros(q.size); dq = np.zeros(q.size); dk = np.zeros(k.size); dv = np.zeros(k.size)
    for pos in range(t):
        for head in range(h):
            qr = (pos * h + head) * d
            kvh = head // (h // kh)
            first = 0 if window == 0 else max(pos + 1 - window, 0)
            ps = list(range(first, pos + 1))
            scores = [sum(q[qr + j] * k[(p * kh + kvh) * d + j] for j in range(d)) / math.sqrt(d) for p in ps]
            m = max(scores)
            z = sum(math.exp(s - m) for s in scores)
            probs = [math.exp(s - m) / z for s in scores]
            dp = [sum(dy[qr + j] * v[(p * kh + kvh) * d + j] for j in range(d)) for p in ps]
            delta = sum(a * b for a, b in zip(probs, dp))
            for j, p in enumerate(ps):
                kr = (p * kh + kvh) * d
                ds = probs[j] * (dp[j] - delta) / math.sqrt(d)
                for col in range(d):
                    out[qr + col] += probs[j] * v[kr + col]
                    dq[qr + col] += ds * k[kr + col]
                    dk[kr + col] += ds * q[qr + col]
                    dv[kr + col] += probs[j] * dy[qr + col]
    return out, dq, dk, dv


@pytest.mark.parametrize("window", [0, 3])
def test_attention_matches_reference_check(window):
    t, h, kh, d = 5, 4, 2, 4
    q = values(t * h * d, 0); k = values(t * kh * d, 3); v = values(t * kh * d, 9); dy = values(t * h * d, 12)
    ref = _attention_reference_check(q, k, v, dy, t, h, kh, d, window)
    o, lse = O.attention_fwd(q.reshape(t, h * d), k.reshape(t, kh * d), v.reshape(t, kh * d), 1, t, h, kh, d, window)
    dq, dk, dv, _ = O.attention_bwd(q.reshape(t, h * d), k.reshape(t, kh * d), v.reshape(t, kh * d), o, lse,
                                    dy.reshape(t, h * d), 1, t, h, kh, d, window)
    for got, exp in zip((o, dq, dk, dv), ref):
        np.testing.assert_allclose(got.ravel(), exp, rtol=1e-12, atol=1e-14)


def test_attention_gqa_equals_repeated_mha_and_fd():
    rng = np.random.default_rng(6)
    B, T, HQ, HK, D = 2, 9, 6, 2, 4
    q = rng.normal(size=(B * T, HQ * D)); k = rng.normal(size=(B * T, HK * D)); v = rng.normal(size=(B * T, HK * D))
    do = rng.normal(size=(B * T, HQ * D))
    o, lse = O.attention_fwd(q, k, v, B, T, HQ, HK, D)
    rep = HQ // HK
    kr = np.repeat(k.reshape(B * T, HK, D), rep, axis=1).reshape(B * T, HQ * D)
    vr = np.repeat(v.reshape(B * T, HK, D), rep, axis=1).reshape(B * T, HQ * D)
    o2, lse2 = O.attention_fwd(q, kr, vr, B, T, HQ, HQ, D)
    np.testing.assert_allclose(o, o2, rtol=1e-13); np.testing.assert_allclose(lse, lse2, rtol=1e-13)
    # first position attends only to itself: o = v, lse = q.k/sqrt(D)
    np.testing.assert_allclose(o.reshape(B * T, HQ, D)[0, 0], v.reshape(B * T, HK, D)[0, 0], rtol=1e-13)
    dq, dk, dv, delta = O.attention_bwd(q, k, v, o, lse, do, B, T, HQ, HK, D)
    np.testing.assert_allclose(delta, (do * o).reshape(-1, D).sum(1), rtol=1e-12)
    f = lambda qq, kk, vv: O.attention_fwd(qq, kk, vv, B, T, HQ, HK, D)[0]
    for e, fd in _fd_vjp(lambda qq: f(qq, k, v), q, do):
        assert abs((dq * e).sum() - fd) < 1e-6 * max(1, abs(fd))
    for e, fd in _fd_vjp(lambda kk: f(q, kk, v), k, do):
        assert abs((dk * e).sum() - fd) < 1e-6 * max(1, abs(fd))
    for e, fd in _fd_vjp(lambda vv: f(q, k, vv), v, do):
        assert abs((dv * e).sum() - fd) < 1e-6 * max(1, abs(fd))


def test_attention_window_covering_sequence_is_causal():
    rng = np.random.default_rng(7)
    B, T, H, D = 1, 6, 2, 4
    q, k, v = (rng.normal(size=(T, H * D)) for _ in range(3))
    a = O.attention_fwd(q, k, v, B, T, H, H, D, 0)
    b = O.attention_fwd(q, k, v, B, T, H, H, D, T)
    np.testing.assert_allclose(a[0], b[0]); np.testing.assert_allclose(a[1], b[1])


# --------------------------------------------------------------- SwiGLU
def test_swiglu_fd():
    rng = np.random.default_rng(8)
    g, u, dy = (rng.normal(size=50) * 3 for _ in range(3))
    dg, du = O.swiglu_bwd(g, u, dy)
    h = O.swiglu_fwd(g, u)
    np.testing.assert_allclose(h, g * u / (1 + np.exp(-g)), rtol=1e-14)
    eps = 1e-6
    np.testing.assert_allclose(dg, dy * (O.swiglu_fwd(g + eps, u) - O.swiglu_fwd(g - eps, u)) / (2 * eps), rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(du, dy * (O.swiglu_fwd(g, u + eps) - O.swiglu_fwd(g, u - eps)) / (2 * eps), rtol=1e-6, atol=1e-9)


# ------------------------------------------------------ CE / embedding
def test_cross_entropy_closed_form_and_fd():
    rng = np.random.default_rng(9)
    x = rng.normal(size=(5, O.VOCAB)) * 3; t = rng.integers(0, 256, 5).astype(np.int32)
    loss, dx = O.cross_entropy(x, t, 0.25)
    m = x.max(1, keepdims=True)
    np.testing.assert_allclose(loss, (m[:, 0] + np.log(np.exp(x - m).sum(1))) - x[np.arange(5), t], rtol=1e-13)
    np.testing.assert_allclose(dx.sum(1), 0.0, atol=1e-14)
    eps = 1e-6
    e = rng.normal(size=x.shape)
    fd = (O.cross_entropy(x + eps * e, t)[0].sum() - O.cross_entropy(x - eps * e, t)[0].sum()) / (2 * eps) * 0.25
    assert abs((dx * e).sum() - fd) < 1e-7


def test_embedding_roundtrip():
    rng = np.random.default_rng(10)
    W = rng.normal(size=(O.VOCAB, 6)); ids = np.array([3, 256, 3, 0], np.int32)
    y = O.embedding_fwd(W, ids)
    np.testing.assert_array_equal(y, W[ids])
    dy = rng.normal(size=(4, 6))
    dW = O.embedding_bwd(dy, ids, O.VOCAB)
    np.testing.assert_allclose(dW[3], dy[0] + dy[2]); np.testing.assert_array_equal(dW[5], 0.0)
    np.testing.assert_allclose(dW[256], dy[1])


# ----------------------------------------------------------------- AdamW
def test_adamw_two_step_closed_form():
    """crates/sejong-train/examples/system_check.rs:135-163: gradient 0.25 then
    0 (the second update sees a zero-filled gradient), lr 1e-3, defaults."""
    b1, b2, eps, wd, lr = 0.9, 0.95, 0.0, 0.1, 0.001
    w0 = 0.3
    w, m, v = np.array([w0]), np.zeros(1), np.zeros(1)
    expected, em, ev = w0, 0.0, 0.0
    for step, g in enumerate([0.25, 0.0]):
        ib1 = 1 / (1 - np.float32(b1) ** np.float32(step + 1))
        ib2 = 1 / (1 - np.float32(b2) ** np.float32(step + 1))
        w, m, v = O.adamw(w, np.array([g]), m, v, lr, b1, b2, eps, wd, ib1, ib2, 1.0)
        em = b1 * em + (1 - b1) * g
        ev = b2 * ev + (1 - b2) * g * g
        expected = expected * (1 - lr * wd) - lr * (em / (1 - b1 ** (step + 1))) / (math.sqrt(ev / (1 - b2 ** (step + 1))) + eps)
    assert abs(w[0] - expected) < 2e-7
    # zero gradient and zero state: the guarded denominator leaves only decay
    w2, _, _ = O.adamw(np.array([1.0]), np.zeros(1), np.zeros(1), np.zeros(1), lr, b1, b2, 0.0, wd, 10.0, 20.0, 1.0)
    assert w2[0] == 1.0 * (1 - lr * wd)


# --------------------------------------------------------------- routing
def test_router_closed_form():
    """Closed-form router check, gpu/examples/hierarchy_check.rs:164-222."""
    logits = np.array([0.2, 1.1, -0.7, 0.6, -0.4, 1.4, -0.1, 0.8, 1.7, 2.1, 0.2, -1.0], np.float32).reshape(4, 3)
    ids, w = O.route_topk(logits, 2)
    x = values(20, 8).reshape(4, 5)
    # combine with expert e scaling its input by (e+1); seed dy = 1
    for row in range(4):
        order = sorted(range(3), key=lambda j: -logits[row, j])
        assert list(ids[row]) == order[:2]
        norm = np.exp(logits[row].astype(np.float64)).sum()
        np.testing.assert_allclose(w[row], np.exp(logits[row, order[:2]].astype(np.float64)) / norm, rtol=1e-12)
        factor = sum(np.exp(float(logits[row, j])) / norm * (j + 1) for j in order[:2])
        s = x[row].sum()
        # d/d weight_k of sum(out) = (e_k+1) * sum(x);  route backward gives dl
        dyk = np.array([[(ids[row, k] + 1) * s for k in range(2)]])
        dl = O.route_topk_bwd(logits[row:row + 1], ids[row:row + 1], w[row:row + 1], dyk)[0]
        for j in range(3):
            up = (j + 1) if j in order[:2] else 0
            np.testing.assert_allclose(dl[j], np.exp(float(logits[row, j])) / norm * s * (up - factor), rtol=1e-10, atol=1e-12)


def test_router_ties_lowest_index_and_pack_order():
    logits = np.array([[1.0, 1.0, 0.5, 1.0], [0.0, 0.0, 0.0, 0.0], [3.0, -1.0, 3.0, 2.0]], np.float32)
    ids, _ = O.route_topk(logits, 2)
    np.testing.assert_array_equal(ids, [[0, 1], [0, 1], [0, 2]])
    tokens, slots, counts = O.route_pack(ids, 4)
    np.testing.assert_array_equal(counts, [3, 2, 1, 0])
    np.testing.assert_array_equal(slots[0, :3], [0, 2, 4]); np.testing.assert_array_equal(tokens[0, :3], [0, 1, 2])
    np.testing.assert_array_equal(slots[1, :2], [1, 3]); np.testing.assert_array_equal(slots[2, :1], [5])


# ----------------------------------------------------------------- model
TINY = dict(d=16, layers=2, hq=4, hk=2, ffn=24, T=6, B=2, eps=1e-6, theta=10000.0)


def _tiny_inputs(cfg, seed=0, std=0.3):
    n = O.model_param_count(cfg["d"], cfg["layers"], cfg["hq"], cfg["hk"], cfg["ffn"])
    rng = np.random.default_rng(seed)
    p = rng.normal(0, std, n)
    ids = rng.integers(0, 256, cfg["T"] * cfg["B"]).astype(np.int32)
    tg = rng.integers(0, 256, cfg["T"] * cfg["B"]).astype(np.int32)
    return p, ids, tg


def test_model_directional_derivative():
    """FD directional derivative of the full loss (system_check.rs:53-107),
    in exact (unrounded) mode so the tolerance can be tight."""
    p, ids, tg = _tiny_inputs(TINY)
    loss, g, _, _ = O.model_fwd_bwd(TINY, p, ids, tg, dtype="none")
    rng = np.random.default_rng(112)
    for _ in range(3):
        d = rng.normal(size=p.size) / math.sqrt(p.size)
        eps = 1e-5
        fd = (O.model_loss(TINY, p + eps * d, ids, tg, "none") - O.model_loss(TINY, p - eps * d, ids, tg, "none")) / (2 * eps)
        an = (g * d).sum()
        assert abs(fd - an) < 1e-7 + 1e-6 * abs(an), (fd, an)


def test_model_per_tensor_fd_and_f32_mode():
    # each parameter tensor separately (catches a wrong gradient on one member)
    cfg = dict(TINY, layers=1)
    p, ids, tg = _tiny_inputs(cfg, seed=3)
    _, g, _, _ = O.model_fwd_bwd(cfg, p, ids, tg, dtype="none")
    d, J, F, V = cfg["d"], cfg["d"] // cfg["hq"] * cfg["hk"], cfg["ffn"], O.VOCAB
    sizes = [V * d, d, d, d * d, d * J, d * J, d * d, d * F, d * F, F * d, d, d * V]
    rng = np.random.default_rng(5)
    off = 0
    for n in sizes:
        e = np.zeros(p.size); e[off:off + n] = rng.normal(size=n)
        eps = 1e-5
        fd = (O.model_loss(cfg, p + eps * e, ids, tg, "none") - O.model_loss(cfg, p - eps * e, ids, tg, "none")) / (2 * eps)
        an = (g * e).sum()
        assert abs(fd - an) < 1e-8 + 1e-6 * abs(an), (off, fd, an)
        off += n
    # f32 storage mode stays within f32 roundoff of the exact mode
    l32, g32, _, _ = O.model_fwd_bwd(cfg, p, ids, tg, dtype="f32")
    lx, gx, _, _ = O.model_fwd_bwd(cfg, p, ids, tg, dtype="none")
    assert abs(l32 - lx) < 1e-5 and np.linalg.norm(g32 - gx) < 1e-4 * np.linalg.norm(gx)


def test_model_causal_prefix_and_batch_separation():
    p, ids, tg = _tiny_inputs(TINY, seed=9)
    _, _, rows, _ = O.model_fwd_bwd(TINY, p, ids, tg, dtype="bf16")
    ids2 = ids.copy(); ids2[4] = (ids2[4] + 1) % 256  # batch 0, position 4
    _, _, rows2, _ = O.model_fwd_bwd(TINY, p, ids2, tg, dtype="bf16")
    T = TINY["T"]
    np.testing.assert_array_equal(rows[:4], rows2[:4])      # causal prefix
    np.testing.assert_array_equal(rows[T:], rows2[T:])      # other sequence
    assert rows[4] != rows2[4]


# ------------------------------------------------------------ MoE FFN
def _moe_case(rng, M=12, d=8, E=4, F=6, std=0.5):
    z = rng.normal(0, 1, (M, d))
    wr = rng.normal(0, 1, (d, E))
    ex = [(rng.normal(0, std, (d, F)), rng.normal(0, std, (d, F)), rng.normal(0, std, (F, d))) for _ in range(E)]
    return z, wr, ex


def test_moe_backward_finite_difference():
    from oracle import moe
    rng = np.random.default_rng(31)
    z, wr, ex = _moe_case(rng)
    K = 2
    R = rng.normal(0, 1, (z.shape[0], z.shape[1]))
    acts = moe.moe_forward(z, wr, ex, K, dtype=None)
    dz, dwr, grads, _, _ = moe.moe_backward(z, wr, ex, acts, R)

    def loss(z_, wr_, ex_):
        a = moe.moe_forward(z_, wr_, ex_, K, dtype=None)
        assert np.array_equal(a["ids"], acts["ids"])  # routing held fixed by the small step
        return float(np.sum(a["update"] * R))

    # routing reads fp32 logits (hierarchy.py:178), so the step must be large
    # against fp32 resolution; the routing stays fixed and O(h^2) is ~1e-6
    h = 1e-3
    def fd(arr, i, f):
        old = arr.flat[i]
        arr.flat[i] = old + h; lp = f()
        arr.flat[i] = old - h; lm = f()
        arr.flat[i] = old
        return (lp - lm) / (2 * h)

    for i in rng.choice(z.size, 6, replace=False):
        assert abs(fd(z, i, lambda: loss(z, wr, ex)) - dz.flat[i]) < 2e-4 * (1 + abs(dz.flat[i]))
    for i in rng.choice(wr.size, 6, replace=False):
        assert abs(fd(wr, i, lambda: loss(z, wr, ex)) - dwr.flat[i]) < 2e-4 * (1 + abs(dwr.flat[i]))
    for e in range(len(ex)):
        for j in range(3):
            W = ex[e][j]
            for i in rng.choice(W.size, 3, replace=False):
                assert abs(fd(W, i, lambda: loss(z, wr, ex)) - grads[e][j].flat[i]) < 2e-4 * (1 + abs(grads[e][j].flat[i]))


def test_moe_single_expert_is_dense_ffn():
    from oracle import moe
    rng = np.random.default_rng(32)
    z, wr, ex = _moe_case(rng, M=20, d=16, E=1, F=24)
    z = O.round_to(z, "bf16")
    ex = [tuple(O.round_to(w, "bf16") for w in ex[0])]
    a = moe.moe_forward(z, wr, ex, 1, dtype="bf16")
    assert np.all(a["w"] == 1.0) and np.all(a["ids"] == 0)
    np.testing.assert_array_equal(a["update"], moe.dense_ffn(z, *ex[0], dtype="bf16"))


# ------------------------------------------------------- parameter VJP
def test_pvjp_indices_match_reference_check_generator():
    """parameter_vjp_check.rs:74-100 builds the expected selection with
    Vec swaps on Rng::new(rng.next_u64()); restated here as text, it must
    equal the kernel-style restatement on the check's default shape."""
    from oracle import pvjp
    n, a, b, rank, frac, block_rows = 67, 71, 97, 33, 0.4, 16
    seed = O.Rng(42).next_u64()
    sel = O.Rng(seed)
    columns = list(range(b))
    for i in range(rank):
        j = i + sel.index(b - i)
        columns[i], columns[j] = columns[j], columns[i]
    blocks = list(range(-(-a // block_rows)))
    count = math.ceil(len(blocks) * frac)
    for i in range(count):
        j = i + sel.index(len(blocks) - i)
        blocks[i], blocks[j] = blocks[j], blocks[i]
    expected_rows = [(i * block_rows + j) if i * block_rows + j < a else -1 for i in blocks[:count] for j in range(block_rows)]
    r, nb, s = pvjp.budget(rank, frac, block_rows, n, a, b)
    assert (r, nb, s) == (33, 5, 2)
    cols, rows, fmap = pvjp.indices(seed, a, b, nb, s, r, block_rows)
    assert cols.tolist() == columns[:rank]
    assert rows.tolist() == expected_rows
    for pos, row in enumerate(rows):
        if row >= 0:
            assert fmap[row] == pos
    assert (fmap >= 0).sum() == (rows >= 0).sum()


def test_pvjp_budget_and_compression_cfg5():
    """cfg5: rank 16, block_rows 32, residual 0.1 over d = 1024 inputs and
    16384 tokens -> 32 blocks, 4 selected; QKV (3 uses) and gate/up (2 uses)
    compress, the single-use attention output and down projections do not."""
    from oracle import pvjp
    n, d, F = 16384, 1024, 2752
    assert pvjp.budget(16, 0.1, 32, n, d, F) == (16, 32, 4)
    assert pvjp.selects_compression(16, 0.1, 32, n, d, 1024, 2 * F, 3)       # query with the widest donor
    assert pvjp.selects_compression(16, 0.1, 32, n, d, F, 2 * F, 2)          # gate
    assert not pvjp.selects_compression(16, 0.1, 32, n, d, d, d, 1)          # attention_output
    assert not pvjp.selects_compression(16, 0.1, 32, n, F, d, d, 1)          # down
    assert not pvjp.selects_compression(16, 1.0, 32, n, d, F, F, 2)          # every block selected
    assert pvjp.issued_gemm(17, 33, 1) == 2 * 32 * 64 * 32


def test_pvjp_basis_orthonormal_span_and_drop():
    from oracle import pvjp
    rng = np.random.default_rng(7)
    n, b, R = 300, 40, 12
    Y = rng.normal(0, 1, (n, b))
    cols = rng.choice(b, R, replace=False)
    eps = pvjp.basis_tolerance(n, R)
    Q = pvjp.basis(Y, cols, eps)
    assert np.abs(Q.T @ Q - np.eye(R)).max() < 1e-12
    Qr, _ = np.linalg.qr(Y[:, cols])
    assert np.abs(Q @ Q.T - Qr @ Qr.T).max() < 1e-12
    Y2 = Y.copy()
    Y2[:, cols[5]] = 2.0 * Y2[:, cols[2]]                                   # dependent column -> dropped
    Q2 = pvjp.basis(Y2, cols, eps)
    assert not Q2[:, 5].any() and abs(np.linalg.norm(Q2[:, 6]) - 1) < 1e-12


def test_pvjp_factored_gradient_all_blocks_is_exact():
    """With every feature row selected (residual weight 1) the factored
    gradient equals X^T D exactly, for any orthonormal Q."""
    from oracle import pvjp
    rng = np.random.default_rng(8)
    n, a, b, R = 50, 20, 9, 6
    X, D = rng.normal(0, 1, (n, a)), rng.normal(0, 1, (n, b))
    Q, _ = np.linalg.qr(rng.normal(0, 1, (n, R)))
    rows = np.arange(a)
    A, E = pvjp.prepare(X, Q, rows, 1, 1)
    coeff = E @ D
    G = pvjp.factored_gradient(a, b, [(A, coeff[:R], coeff[R:], np.arange(a), 1.0)])
    assert np.abs(G - X.T @ D).max() < 1e-10
    # a subset: selected rows carry X^T D, the others the low-rank part
    rows = np.array([3, 4, 5, -1])
    fmap = np.full(a, -1); fmap[[3, 4, 5]] = [0, 1, 2]
    A, E = pvjp.prepare(X, Q, rows, 2, 1)
    coeff = E @ D
    G = pvjp.factored_gradient(a, b, [(A, coeff[:R], coeff[R:], fmap, 1.0)])
    low = A @ (Q.T @ D)
    assert np.abs(G[0] - low[0]).max() < 1e-10
    assert np.abs(G[3] - (low[3] + 2 * (X[:, 3] - Q @ A[3]) @ D)).max() < 1e-10


def test_pvjp_update_closed_form():
    from oracle import pvjp
    W = np.array([[1.0, -2.0], [0.5, 0.25]]); G = np.array([[0.1, 0.2], [-0.3, 0.4]])
    lr, clip, wd = 0.01, 0.7, 0.02
    LR = float(np.float32(np.float32(lr) * np.float32(clip))); DEC = float(np.float32(np.float32(lr) * np.float32(wd)))
    np.testing.assert_allclose(pvjp.factored_update(W, G, lr, clip, wd, True), W * (1 - DEC) - LR * G, rtol=0, atol=0)
    np.testing.assert_allclose(pvjp.factored_update(W, G, lr, clip, wd, False), W - LR * G, rtol=0, atol=0)


# --------------------------------------------------------- golden fixtures
@pytest.mark.parametrize("name", ["cfg1_step", "attention_values", "router", "pvjp_selection", "moe_ffn_tiny"])
def test_golden_fixture_reproduces(name):
    """Every committed fixture is what the pinned oracle computes now."""
    import os
    from tests.golden import make_golden as G
    ref = np.load(os.path.join(os.path.dirname(G.__file__), name + ".npz"), allow_pickle=False)
    got = G.CASES[name]()
    assert sorted(ref.files) == sorted(got)
    for key in ref.files:
        a, b = np.asarray(got[key]), ref[key]
        if a.dtype.kind in "iu":
            np.testing.assert_array_equal(a, b, err_msg=key)
        else:
            np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-14, err_msg=key)


def test_model_backward_projection_dys():
    """The per-layer output gradients of the projection Matmul nodes (the dY
    a parameter VJP contracts with): X^T dY reproduces each projection's
    FD-pinned weight gradient (q and k pre-RoPE, as the Matmul node values)."""
    cfg = dict(TINY)
    p, ids, tg = _tiny_inputs(cfg, seed=4)
    acts = O.model_forward(cfg, p, ids, dtype="none")
    loss, g, _, dys = O.model_backward(cfg, p, acts, ids, tg, dtype="none", want_dys=True)
    lr, gr, _ = O.model_backward(cfg, p, acts, ids, tg, dtype="none")
    assert loss == lr and np.array_equal(g, gr)
    d, J, F, V, M = cfg["d"], cfg["d"] // cfg["hq"] * cfg["hk"], cfg["ffn"], O.VOCAB, cfg["T"] * cfg["B"]
    A, off = {}, 0
    for name, layer, size in O.acts_layout(cfg):
        A[(name, layer)] = acts[off:off + size]
        off += size
    off = V * d
    for l in range(cfg["layers"]):
        z, z2 = A[("z", l)].reshape(M, d), A[("z2", l)].reshape(M, d)
        off += 2 * d
        for name, X, n in (("q", z, d), ("k", z, J), ("v", z, J)):
            np.testing.assert_allclose((X.T @ dys[l][name]).ravel(), g[off:off + d * n], rtol=1e-9, atol=1e-14)
            off += d * n
        off += d * d
        for name in ("gate", "up"):
            np.testing.assert_allclose((z2.T @ dys[l][name]).ravel(), g[off:off + d * F], rtol=1e-9, atol=1e-14)
            off += d * F
        off += F * d


# ------------------------------------------------------ hierarchy patches
def test_patch_maps_closed_forms():
    from oracle import hierarchy as OH
    B, T, d, P = 2, 10, 3, 4     # patches of 4, 4, 2 positions
    x = np.arange(B * T * d, dtype=np.float64).reshape(B * T, d)
    y = OH.patch_pool(x, B, T, P).reshape(B, 3, d)
    xr = x.reshape(B, T, d)
    np.testing.assert_array_equal(y[:, 0], xr[:, 0:4].mean(1))
    np.testing.assert_array_equal(y[:, 2], xr[:, 8:10].mean(1))   # partial patch: its own count
    np.testing.assert_array_equal(OH.patch_pool(np.full((B * T, d), 0.75), B, T, 16), 0.75 * np.ones((B, d)))  # patch > t
    z = np.arange(B * 3 * d, dtype=np.float64).reshape(B * 3, d)
    bos = np.array([-1.0, -2.0, -3.0])
    yb = OH.patch_broadcast(z, bos, B, T, P).reshape(B, T, d)
    np.testing.assert_array_equal(yb[:, :4], np.broadcast_to(bos, (B, 4, d)))
    np.testing.assert_array_equal(yb[:, 4:8], np.broadcast_to(z.reshape(B, 3, d)[:, 0:1], (B, 4, d)))
    np.testing.assert_array_equal(yb[:, 8:], np.broadcast_to(z.reshape(B, 3, d)[:, 1:2], (B, 2, d)))


@pytest.mark.parametrize("T,P", [(10, 4), (12, 4), (5, 8), (7, 1)])
def test_patch_maps_adjoints(T, P):
    from oracle import hierarchy as OH
    rng = np.random.default_rng(T * 10 + P)
    B, d = 3, 5
    NP = -(-T // P)
    x = rng.normal(size=(B * T, d)).astype(np.float32).astype(np.float64)
    yv = rng.normal(size=(B * NP, d)).astype(np.float32).astype(np.float64)
    lhs = np.sum(OH.patch_pool(x, B, T, P) * yv)
    rhs = np.sum(x * OH.patch_pool_backward(yv, B, T, P))
    assert abs(lhs - rhs) < 1e-5 * (1 + abs(lhs))
    z = rng.normal(size=(B * NP, d)).astype(np.float32).astype(np.float64)
    bos = rng.normal(size=d).astype(np.float32).astype(np.float64)
    dy = rng.normal(size=(B * T, d)).astype(np.float32).astype(np.float64)
    dx, dbos = OH.patch_broadcast_backward(dy, B, T, P)
    lhs = np.sum(OH.patch_broadcast(z, bos, B, T, P) * dy)
    rhs = np.sum(z * dx) + np.sum(bos * dbos)
    assert abs(lhs - rhs) < 1e-5 * (1 + abs(lhs))


def test_model_backward_hidden_matches_lm_head():
    """The body backward from a given final-norm gradient reproduces the
    FD-pinned full backward when fed the LM head's own dh, with the
    embedding gradient formed from the returned embedding-output gradient."""
    cfg = dict(TINY)
    p, ids, tg = _tiny_inputs(cfg, seed=6)
    acts = O.model_forward(cfg, p, ids, dtype="none")
    loss, g, _ = O.model_backward(cfg, p, acts, ids, tg, dtype="none")
    d, M, V = cfg["d"], cfg["T"] * cfg["B"], O.VOCAB
    A, off = {}, 0
    for name, layer, size in O.acts_layout(cfg):
        A[(name, layer)] = acts[off:off + size]
        off += size
    logits = A[("logits", -1)].reshape(M, V)
    _, dlog = O.cross_entropy(logits, tg, float(np.float32(1.0) / np.float32(M)))  # the f32 seed
    wout = p[-d * V:].reshape(d, V)
    dh = dlog @ wout.T
    gh, demb = O.model_backward_hidden(cfg, p, acts, dh, dtype="none")
    n = g.size
    np.testing.assert_allclose(gh[V * d:n - d * V], g[V * d:n - d * V], rtol=1e-10, atol=1e-15)
    np.testing.assert_allclose(O.embedding_bwd(demb, ids, V).ravel(), g[:V * d], rtol=1e-10, atol=1e-15)


def _hier_cfg(window=6):
    return dict(d=32, layers=1, hq=4, hk=2, ffn=48, T=16, B=2, P=4, window=window, de=16, le=1, he=2, fe=40,
                dd=16, ld=2, hd=2, fd=24, eps=1e-6, theta=10000.0)


def test_hierarchy_model_gradient_finite_difference():
    """The hierarchical model's composed backward (encoder, pool,
    encoder_to_global, global stack, global_to_decoder of patches and BOS,
    broadcast, encoder_to_decoder, decoder, output_projection, final norm,
    head) against central differences of its own FP64 loss, for entries of
    every glue tensor and of each stage (window 6 < T = 16)."""
    from oracle import hierarchy as H
    cfg = _hier_cfg()
    table, total = H._offsets(cfg)
    rng = np.random.default_rng(5)
    p = rng.normal(0, 0.3, total)
    for name, (o, shape) in table.items():
        if name.endswith("norm"):
            p[o:o + int(np.prod(shape))] = 1.0 + rng.normal(0, 0.1, int(np.prod(shape)))
    M = cfg["B"] * cfg["T"]
    ids = rng.integers(0, 256, M).astype(np.int32)
    tg = rng.integers(0, 256, M).astype(np.int32)
    acts = H.model_forward(cfg, p, ids, "none")
    loss, g = H.model_backward(cfg, p, acts, ids, tg, "none")
    assert abs(loss - H.model_loss(cfg, p, ids, tg)) < 1e-12
    names = ["embedding", "encoder.0.query", "encoder.0.down", "encoder_norm", "encoder_to_global",
             "encoder_to_decoder", "global_to_decoder", "global_bos", "global_norm", "layers.0.key",
             "layers.0.up", "decoder.1.value", "decoder.0.gate", "decoder_norm", "output_projection",
             "final_norm", "output", "encoder.0.attention_norm", "decoder.1.ffn_norm"]
    h = 1e-5
    worst = 0.0
    for name in names:
        o, shape = table[name]
        n = int(np.prod(shape))
        idx = [o + i for i in rng.choice(n, size=min(n, 3), replace=False)]
        if name == "embedding":
            idx = [o + int(ids[0]) * cfg["de"] + 1, o + int(ids[5]) * cfg["de"] + 3]
        for i in idx:
            pp, pm = p.copy(), p.copy()
            pp[i] += h
            pm[i] -= h
            fd = (H.model_loss(cfg, pp, ids, tg) - H.model_loss(cfg, pm, ids, tg)) / (2 * h)
            err = abs(fd - g[i]) / (abs(fd) + 1e-6)
            worst = max(worst, err)
            assert err < 1e-4, (name, i, fd, g[i])
    # input_projection only serves injected inputs: zero gradient
    o, shape = table["input_projection"]
    assert not np.any(g[o:o + int(np.prod(shape))])
    print(f"[hierarchy] worst FD relative error {worst:.2e}")


def test_hierarchy_window_and_stage_reduce_to_dense_blocks():
    """A stage with a window at least its sequence is the dense model's
    body: the stage forward's activations equal or_model_forward's for the
    same blocks and input embedding, and a window shorter than the sequence
    changes them (it is applied)."""
    cfg = dict(d=16, layers=2, hq=2, hk=1, ffn=24, T=12, B=2, eps=1e-6, theta=10000.0)
    rng = np.random.default_rng(9)
    n = O.model_param_count(16, 2, 2, 1, 24)
    p = rng.normal(0, 0.3, n)
    M = 24
    ids = rng.integers(0, 256, M).astype(np.int32)
    acts = O.model_forward(cfg, p, ids, "none")
    V, d = O.VOCAB, 16
    body = p[V * d:n - d * V]                    # layers + final norm (the stage layout)
    x0 = p[:V * d].reshape(V, d)[ids]
    st = O.stage_forward(dict(cfg, window=12), body, x0, "none")
    np.testing.assert_allclose(st, acts[:st.size], rtol=0, atol=1e-12)
    st_w = O.stage_forward(dict(cfg, window=5), body, x0, "none")
    assert np.max(np.abs(st_w - st)) > 1e-3
    # the stage backward equals the dense body backward through model_backward_hidden
    dz = rng.normal(0, 1, (M, d))
    g_dense, demb = O.model_backward_hidden(cfg, p, acts, dz, "none")
    g_stage, dx = O.stage_backward(dict(cfg, window=0), body, st, dz, "none")
    np.testing.assert_allclose(g_stage, g_dense[V * d:n - d * V], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dx, demb, rtol=1e-12, atol=1e-12)


def _moe_model_cfg(E=3, K=2):
    return dict(d=16, layers=2, hq=2, hk=1, E=E, K=K, fe=12, T=8, B=2, eps=1e-6, theta=10000.0)


def _moe_params(cfg, rng):
    from oracle import moe
    table, total = moe._offsets(cfg)
    p = rng.normal(0, 0.3, total)
    for name, (o, shape) in table.items():
        if name.endswith("norm"):
            p[o:o + int(np.prod(shape))] = 1.0 + rng.normal(0, 0.1, int(np.prod(shape)))
    return table, p


def test_moe_model_single_expert_is_dense_model():
    """E = 1, K = 1: every routing weight is exactly 1, so the MoE model is
    the dense model with gate / up / down = expert 0's: loss and gradients
    equal the dense C oracle's (exact FP64 and bf16 storage), and the
    router's gradient is exactly 0."""
    from oracle import moe
    cfg = _moe_model_cfg(E=1, K=1)
    rng = np.random.default_rng(17)
    table, p = _moe_params(cfg, rng)
    keep = np.ones(p.size, bool)
    for l in range(cfg["layers"]):
        o, shape = table[f"layers.{l}.router"]
        keep[o:o + int(np.prod(shape))] = False
    dense = p[keep]
    dcfg = dict(d=16, layers=2, hq=2, hk=1, ffn=12, T=8, B=2, eps=1e-6, theta=10000.0)
    assert dense.size == O.model_param_count(16, 2, 2, 1, 12)
    M = 16
    ids = rng.integers(0, 256, M).astype(np.int32)
    tg = rng.integers(0, 256, M).astype(np.int32)
    for dtype, tol in (("none", 1e-11), ("bf16", 1e-11)):
        acts = moe.model_forward(cfg, p, ids, dtype)
        loss, g, routing = moe.model_backward(cfg, p, acts, ids, tg, dtype)
        dloss, dg, _, _ = O.model_fwd_bwd(dcfg, dense, ids, tg, dtype)
        assert abs(loss - dloss) <= tol * abs(dloss), (dtype, loss, dloss)
        np.testing.assert_allclose(g[keep], dg, rtol=tol, atol=tol * np.abs(dg).max())
        assert not np.any(g[~keep])
        for ids_l, w_l, counts, _, _ in routing:
            assert np.all(ids_l == 0) and np.all(w_l == 1.0) and counts[0] == M


def test_moe_model_gradient_finite_difference():
    """The composed MoE model backward (head, final norm, per layer the
    MoE FFN with the router, ffn norm, attention, QKV, attention norm,
    embedding) against central differences of its own exact FP64 loss for
    entries of every tensor kind (routing held fixed: no top-k swap within
    the step)."""
    from oracle import moe
    cfg = _moe_model_cfg()
    rng = np.random.default_rng(23)
    table, p = _moe_params(cfg, rng)
    M = cfg["B"] * cfg["T"]
    ids = rng.integers(0, 256, M).astype(np.int32)
    tg = rng.integers(0, 256, M).astype(np.int32)
    acts = moe.model_forward(cfg, p, ids, "none")
    loss, g, routing = moe.model_backward(cfg, p, acts, ids, tg, "none")
    assert abs(loss - moe.model_loss(cfg, p, ids, tg)) < 1e-12
    assert all(np.all(r[2] > 0) for r in routing)          # every expert receives rows
    names = ["embedding", "layers.0.attention_norm", "layers.0.query", "layers.1.key", "layers.0.value",
             "layers.1.attention_output", "layers.0.ffn_norm", "layers.0.experts.0.gate", "layers.1.experts.2.up",
             "layers.0.experts.1.down", "layers.0.router", "layers.1.router", "final_norm", "output"]
    h = 1e-5
    worst = 0.0
    for name in names:
        o, shape = table[name]
        n = int(np.prod(shape))
        idx = [o + i for i in rng.choice(n, size=min(n, 3), replace=False)]
        if name == "embedding":
            idx = [o + int(ids[0]) * cfg["d"] + 1, o + int(ids[5]) * cfg["d"] + 3]
        for i in idx:
            pp, pm = p.copy(), p.copy()
            pp[i] += h
            pm[i] -= h
            fd = (moe.model_loss(cfg, pp, ids, tg) - moe.model_loss(cfg, pm, ids, tg)) / (2 * h)
            err = abs(fd - g[i]) / (abs(fd) + 1e-6)
            worst = max(worst, err)
            assert err < 1e-4, (name, i, fd, g[i])
    print(f"[moe model] worst FD relative error {worst:.2e}")


def test_sum_squares_against_exact_sums():
    """or_sum_squares (the FP64 gradient norm, kernels.py:265-287) against
    sums it cannot share code with: the closed form sum_{i<=n} i^2 =
    n(n+1)(2n+1)/6 (exact in FP64 at this n), math.fsum of the squares
    (correctly rounded) on random, large-magnitude and tiny vectors, and
    numpy's dot."""
    n = 100000
    i = np.arange(1, n + 1, dtype=np.float64)
    assert O.sum_squares(i) == n * (n + 1) * (2 * n + 1) // 6
    rng = np.random.default_rng(7)
    for g in (rng.normal(0, 1, 50001), rng.normal(0, 1e100, 4097) * rng.integers(0, 2, 4097),
              rng.normal(0, 1e-150, 1000), np.float32(rng.normal(0, 3, 9999)).astype(np.float64)):
        exact = math.fsum(float(v) * float(v) for v in g)
        got = O.sum_squares(g)
        assert abs(got - exact) <= 1e-12 * exact, (got, exact)
        assert abs(got - float(np.dot(g, g))) <= 1e-12 * exact
    assert O.sum_squares(np.zeros(0)) == 0.0
    assert O.sum_squares(np.array([-3.0, 4.0])) == 25.0


def test_pvjp_basis_tolerance_hand_values():
    """pvjp.basis_tolerance against parameter_vjp.rs:214-220 evaluated in
    exact rational arithmetic: operations = rows (4 rank + 1), roundoff =
    operations * f32::EPSILON / 2 = operations / 2^24, tolerance = roundoff /
    (1 - roundoff) = operations / (2^24 - operations) while roundoff < 1,
    else infinity, then min(., f32::MAX) as f32."""
    from fractions import Fraction

    from oracle import pvjp
    f32max = float(np.finfo(np.float32).max)

    def by_hand(rows, rank):
        ops = rows * (4 * rank + 1)
        if ops >= 2 ** 24:                       # roundoff >= 1 -> inf -> FLT_MAX
            return np.float32(f32max)
        return np.float32(float(Fraction(ops, 2 ** 24 - ops)))

    # literal values: 1 / (2^24 - 1), 4355 / 16772861 (the check program's 67 x 16)
    assert pvjp.basis_tolerance(1, 0) == np.float32(1.0 / 16777215.0)
    assert pvjp.basis_tolerance(67, 16) == np.float32(4355.0 / 16772861.0)
    for rows, rank in [(67, 16), (16384, 16), (4096, 16), (97, 33), (1, 1), (8192, 64), (255, 0)]:
        assert pvjp.basis_tolerance(rows, rank) == by_hand(rows, rank), (rows, rank)
    # roundoff exactly 1 (rows 2^24, rank 0) and beyond: the infinity branch clamps to FLT_MAX
    assert pvjp.basis_tolerance(2 ** 24, 0) == np.float32(f32max)
    assert pvjp.basis_tolerance(1 << 20, 4) == np.float32(f32max)
    # one operation short of 1: the largest finite tolerance, 2^24 - 1
    assert pvjp.basis_tolerance(2 ** 24 - 1, 0) == np.float32(16777215.0)


def test_blake3_published_digests_and_reference_fingerprints():
    """oracle/blake3.py against the BLAKE3 specification's digests of the
    empty input and "abc" (one block, one chunk), and, where the reference
    checkout is present, against the corpus fingerprints its measurement
    recorded (multi-chunk trees: docs/measurements/2026-11-01/
    rx6600-learning-window.json:2111,2119).  A wrong rotation, message
    permutation, flag or tree split fails one of them."""
    import os
    from oracle import blake3 as B3
    assert B3.blake3(b"").hex() == "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"
    assert B3.blake3(b"abc").hex() == "6437b3ac38465133ffb63b75273a8db548c558465d79db03fd359c6cd5bd9d85"
    d = "/root/reference/docs/measurements/2026-11-01/"
    if os.path.exists(d + "train.txt"):
        with open(d + "train.txt", "rb") as f:
            assert B3.corpus_fingerprint([f.read()]) == \
                "b96cc76f31fa0a61e840635e05d1ceea137d68329cbe2d20504b8f34d371943f"
        with open(d + "validation.txt", "rb") as f:
            assert B3.corpus_fingerprint([f.read()]) == \
                "9a1409d8fd61e18c2ca1fef712488fbe776e90f3c10fd9a9b88d9eb11503d16e"


def _production_matmuls(expert_rows=256):
    """The parameter products of one training step of the reference's
    production model (configs/sejong.toml: hierarchical with 8-byte patches;
    encoder and decoder 2 x d128 with 2 heads and FFN 384, window
    128; global 8 x d512, 8 query / 4 KV heads, 4 SwiGLU experts of 384 with
    top-2 routing; batch 8 x 512 bytes), in graph order, as (input id, rows,
    input width, output width): architecture.rs:200-247 (Block::apply) and
    368-393 (hidden_from_encoded).  Every expert sees `expert_rows` of the 512
    patches (top-2 of 4: 256 on average; never all 512)."""
    Ml, Mg = 8 * 512, 8 * 512 // 8
    out, nid = [], [0]

    def new():
        nid[0] += 1
        return nid[0]

    def local():
        for _ in range(2):
            z, o, z2, h = new(), new(), new(), new()
            out.extend([(z, Ml, 128, 128)] * 3)                       # q, k, v (2 heads = 2 KV heads)
            out.append((o, Ml, 128, 128))                             # attention_output
            out.extend([(z2, Ml, 128, 384)] * 2)                      # gate, up
            out.append((h, Ml, 384, 128))                             # down

    local()                                                           # encoder
    out.append((new(), Mg, 128, 512))                                 # encoder_to_global (pooled)
    for _ in range(8):                                                # global stage over the patches
        z, o, z2 = new(), new(), new()
        out.extend([(z, Mg, 512, 512), (z, Mg, 512, 256), (z, Mg, 512, 256)])
        out.append((o, Mg, 512, 512))
        out.append((z2, Mg, 512, 4))                                  # router
        for _ in range(4):
            xe, he = new(), new()
            out.extend([(xe, expert_rows, 512, 384)] * 2)             # expert gate, up (gathered rows)
            out.append((he, expert_rows, 384, 512))                   # expert down
    out.append((new(), Mg, 512, 128))                                 # global_to_decoder (latent)
    out.append((new(), 1, 512, 128))                                  # global_to_decoder (BOS row)
    out.append((new(), Ml, 128, 128))                                 # encoder_to_decoder
    local()                                                           # decoder
    out.append((new(), Ml, 128, 512))                                 # output_projection
    out.append((new(), Ml, 512, 257))                                 # output head (fp32 master)
    return out


def test_pvjp_graph_statistics_match_reference_production_record():
    """The compression decisions and grouping (graph.rs:551-566, 915-1005,
    with selects_compression and budget of parameter_vjp.rs:85-130) on the
    reference's production configuration give the statistics its measurement
    recorded for every one of its 64 steps: 44 compressed and 126 dense
    matrices, 2 basis groups and 16 projection groups
    (docs/measurements/2026-11-01-architecture-fit/applied.json,
    parameter_vjp_statistics; rank 16, residual_fraction 0.25, block_rows
    32).  The 16 groups are the 8 global q|k|v groups (512 patches) and the
    encoder's and decoder's 2 q|k|v and 2 gate|up groups (4096 bytes: a
    second token basis); single-use products and the expert products (fewer
    routed rows than input columns) stay dense.  Also at the routing
    extremes an expert can reach (any count below 512 rows)."""
    import os
    from oracle import pvjp
    want = dict(compressed_matrices=44, dense_matrices=126, basis_groups=2, projection_groups=16)
    for rows in (256, 1, 511):
        mm = _production_matmuls(rows)
        assert len(mm) == 170
        assert pvjp.graph_statistics(mm, 16, 0.25, 32) == want, rows
    rec = "/root/reference/docs/measurements/2026-11-01-architecture-fit/applied.json"
    if os.path.exists(rec):
        import json
        steps = json.load(open(rec))["runs"][0]["measured_step_records"]
        assert len(steps) == 64 and all(s["parameter_vjp_statistics"] == want for s in steps)
    # the record constrains the inputs: other settings give other counts
    # (all blocks selected: nothing compresses; 128-row blocks: the local
    # stages' 128 features form one block, fully selected; every expert
    # reaching 512 rows: its gate|up group forms too)
    mm = _production_matmuls(256)
    assert pvjp.graph_statistics(mm, 16, 1.0, 32)["compressed_matrices"] == 0
    assert pvjp.graph_statistics(mm, 16, 0.25, 128)["compressed_matrices"] == 24
    assert pvjp.graph_statistics(_production_matmuls(512), 16, 0.25, 32)["projection_groups"] > 16
