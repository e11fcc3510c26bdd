"""KV-cache inference and evaluation (Model::new_cache / forward_cached,
model lib.rs:36-50 and 359-394, architecture.rs:428-533 and 758-799;
benchmark.rs:71-171) on the GPU.

Cached logits are compared with the model's own full-sequence forward: the
reference's system check requires max |cached - full| < 1e-4 over every
position of an fp32 model (crates/sejong-train/examples/system_check.rs:
38-52); the cached kernels compute each row with the full forward's
operations, so the bf16 models are held to the same bound (and are in fact
bit-identical).  The full forward itself is pinned against the FP64 oracle
(fp32 end to end; bf16 loss within 1e-3), and the evaluation BPB is the
oracle's mean loss / ln 2 on the same Corpus batches."""
import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import dev, empty, rnd, sync, zeros

pytestmark = pytest.mark.gpu

TOL = 1e-4  # system_check.rs:48-51
SYSTEM_TOKENS = [256, 83, 101, 106, 111, 110, 103, 32, 234, 184, 128]


def _model(mc, tc, seed=42):
    from sejong_amd.model import Model, init_params
    params = init_params(mc, std=0.02, seed=seed)
    m = Model(mc, tc)
    m.set_params(params)
    return m, params


def _ocfg(mc, tc):
    return dict(d=mc.width, layers=mc.layers, hq=mc.heads, hk=mc.kv, ffn=mc.ffn_width, T=tc.sequence, B=tc.batch,
                eps=mc.norm_epsilon, theta=mc.rope_theta)


@pytest.mark.parametrize("T,L,window", [(256, 0, 0), (256, 100, 0), (256, 255, 0), (192, 37, 0), (256, 70, 50)])
def test_cached_attention_op_bf16_matches_full_rows(T, L, window):
    """sj_attention_fwd_cached (MFMA layout) against rows L.. of the full
    causal (windowed) attention of the same q|k|v: bit for bit."""
    from sejong_amd import _native as N
    N.load()
    api = N.api
    HQ, HK, Dh = 6, 2, 64
    d, J = HQ * Dh, HK * Dh
    NQ = d + 2 * J
    rng = np.random.default_rng(T + L + window)
    qkv = rnd((T, NQ), "bf16", rng)
    QKV = dev(qkv, "bf16")
    O1, LSE, LSET = empty(T * d, "bf16"), empty(T * HQ), empty(HQ * T)
    api.sj_attention_fwd_tt(None, QKV.p, NQ, T, 1, T, HQ, HK, Dh, window, O1.p, d, LSE.p, LSET.p, None, 0)
    q, k, v = qkv[L:, :d], qkv[:, d:d + J], qkv[:, d + J:]
    Q, K, V = dev(np.ascontiguousarray(q), "bf16"), dev(np.ascontiguousarray(k), "bf16"), dev(np.ascontiguousarray(v), "bf16")
    O2 = empty((T - L) * d, "bf16")
    api.sj_attention_fwd_cached(None, Q.p, d, K.p, V.p, J, T, N.SJ_BF16, T - L, L, HQ, HK, Dh, window, O2.p, d)
    sync()
    full = O1.host().reshape(T, d)
    np.testing.assert_array_equal(O2.host().reshape(T - L, d), full[L:])
    # and the full kernel against the FP64 oracle (sanity of the reference rows)
    ref, _ = O.attention_fwd(qkv[:, :d], k, v, 1, T, HQ, HK, Dh, window=window)
    assert np.max(np.abs(full - ref)) < 2e-2


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_cached_attention_op_rows_kernel(dtype):
    """The row kernel's cached form (fp32, or head_dim != 64) against the
    full row kernel's rows."""
    from sejong_amd import _native as N
    N.load()
    api = N.api
    T, L, HQ, HK, Dh = 40, 13, 4, 2, 32
    d, J = HQ * Dh, HK * Dh
    rng = np.random.default_rng(5)
    q, k, v = rnd((T, d), dtype, rng), rnd((T, J), dtype, rng), rnd((T, J), dtype, rng)
    dt = N.SJ_F32 if dtype == "f32" else N.SJ_BF16
    Q, K, V = dev(q, dtype), dev(k, dtype), dev(v, dtype)
    O1, LSE = empty(T * d, dtype), empty(T * HQ)
    api.sj_attention_fwd(None, Q.p, d, K.p, J, V.p, J, O1.p, d, LSE.p, dt, 1, T, HQ, HK, Dh, 0)
    Q2 = dev(np.ascontiguousarray(q[L:]), dtype)
    O2 = empty((T - L) * d, dtype)
    api.sj_attention_fwd_cached(None, Q2.p, d, K.p, V.p, J, T, dt, T - L, L, HQ, HK, Dh, 0, O2.p, d)
    sync()
    np.testing.assert_array_equal(O2.host().reshape(T - L, d), O1.host().reshape(T, d)[L:])


def test_fp32_system_check_cached_vs_full_and_oracle():
    """system_check.rs:35-52 at the cfg1 block shape: one token at a time
    through the cache, every position's logits against the full forward
    (< 1e-4) and against the FP64 oracle."""
    from sejong_amd.model import ModelConfig, TrainConfig
    T = len(SYSTEM_TOKENS)
    mc = ModelConfig(width=128, layers=2, heads=4, kv_heads=2, ffn_width=384, context=64, norm_epsilon=1e-6,
                     precision="f32", seed=97)
    tc = TrainConfig(sequence=T, batch=1)
    m, params = _model(mc, tc, seed=97)
    try:
        ids = np.array(SYSTEM_TOKENS, np.int32)
        targets = np.array(SYSTEM_TOKENS[1:] + [46], np.int32)
        m.set_batch(ids, targets)
        loss = m.forward()
        full = m.logits()
        lref, _, _, lg = O.model_fwd_bwd(_ocfg(mc, tc), params.astype(np.float64), ids, targets, "f32",
                                         want_logits=True)
        assert abs(loss - lref) < 1e-5 * abs(lref)
        assert np.max(np.abs(full - lg)) < 1e-5
        cache = m.new_cache()
        worst = 0.0
        for end in range(1, T + 1):
            got = m.forward_cached(ids[end - 1:end], cache)
            worst = max(worst, float(np.max(np.abs(got - full[end - 1]))))
        print(f"[infer] fp32 cached vs full max abs error {worst:.3e}")
        assert worst < TOL and cache.length == T
        # reset and a prefill of the whole prefix give the same last row
        cache.reset()
        got = m.forward_cached(ids, cache)
        assert np.max(np.abs(got - full[-1])) < TOL
        cache.close()
    finally:
        m.close()


def test_bf16_cfg2_prefill_decode_bit_exact():
    """The cfg2 model (6 layers, d384, GQA 6/2) on one 512-byte sequence:
    prefill in uneven chunks (query blocks straddling 64-row blocks), then
    teacher-forced decode; every chunk's last logits equal the full
    forward's row."""
    from sejong_amd.model import config
    mc, tc = config("cfg2")
    tc.batch = 1
    m, params = _model(mc, tc)
    try:
        rng = np.random.default_rng(11)
        ids = rng.integers(0, 257, tc.sequence).astype(np.int32)
        from sejong_amd.benchmark import full_logits
        full = full_logits(m, ids)
        cache = m.new_cache()
        pos, worst = 0, 0.0
        for n in [1, 63, 64, 100, 2, 200, 66] + [1] * 16:
            got = m.forward_cached(ids[pos:pos + n], cache)
            pos += n
            worst = max(worst, float(np.max(np.abs(got - full[pos - 1]))))
        assert pos == tc.sequence == cache.length
        print(f"[infer] bf16 cfg2 cached vs full max abs error {worst:.3e}")
        assert worst <= TOL
        from sejong_amd import _native as N
        with pytest.raises(N.SejongError, match="context limit"):
            m.forward_cached(ids[:1], cache)
        cache.reset()
        with pytest.raises(N.SejongError, match="bytes or EOS"):
            m.forward_cached(np.array([257]), cache)
        cache.close()
    finally:
        m.close()


def test_moe_cached_vs_full():
    """Routed experts in the cached blocks: token-by-token decode after a
    prefill, against the full forward."""
    from sejong_amd.model import ExpertConfig, ModelConfig, TrainConfig
    mc = ModelConfig(width=256, layers=2, heads=4, kv_heads=2, ffn_width=256, context=128, precision="bf16",
                     experts=ExpertConfig(count=4, top_k=2, ffn_width=256))
    tc = TrainConfig(sequence=128, batch=1)
    m, _ = _model(mc, tc)
    try:
        ids = np.random.default_rng(3).integers(0, 256, 128).astype(np.int32)
        from sejong_amd.benchmark import full_logits
        full = full_logits(m, ids)
        cache = m.new_cache()
        got = m.forward_cached(ids[:100], cache)
        worst = float(np.max(np.abs(got - full[99])))
        for p in range(100, 128):
            got = m.forward_cached(ids[p:p + 1], cache)
            worst = max(worst, float(np.max(np.abs(got - full[p]))))
        print(f"[infer] MoE cached vs full max abs error {worst:.3e}")
        assert worst <= TOL
        cache.close()
    finally:
        m.close()


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_evaluate_bpb_matches_oracle(tmp_path, precision):
    """evaluate (benchmark.rs:71-99) on a corpus of three documents: BPB =
    the oracle's mean loss of the same Corpus::batch draws / ln 2 (fp32 end
    to end 1e-6; bf16 storage within the 1e-3 loss gate)."""
    from sejong_amd.benchmark import evaluate
    from sejong_amd.corpus import Corpus
    from sejong_amd.model import ModelConfig, TrainConfig
    from sejong_amd.rng import Rng
    rng = np.random.default_rng(9)
    for i, n in enumerate([3000, 17, 900]):
        (tmp_path / f"d{i}.txt").write_bytes(rng.integers(32, 127, n, dtype=np.uint8).tobytes())
    corpus = Corpus.open(tmp_path)
    mc = ModelConfig(width=128, layers=2, heads=4, kv_heads=2, ffn_width=256, context=128, norm_epsilon=1e-6,
                     precision=precision)
    tc = TrainConfig(sequence=128, batch=2, seed=123)
    m, params = _model(mc, tc)
    try:
        bpb = evaluate(m, corpus, 3)
        r = Rng(123)
        losses = []
        for _ in range(3):
            ids, tg = corpus.batch(r, tc.batch, tc.sequence)
            losses.append(O.model_loss(_ocfg(mc, tc), params.astype(np.float64), ids, tg, precision))
        ref = float(np.mean(losses)) / math.log(2.0)
        print(f"[infer] {precision} BPB {bpb:.6f} oracle {ref:.6f}")
        assert abs(bpb - ref) < (1e-6 if precision == "f32" else 1e-3) * ref
    finally:
        m.close()


def test_cached_measurement_report(tmp_path):
    """cached_measurement (benchmark.rs:113-171) at the cfg2 shape: the
    report's error field is the largest |cached - full| of the last token."""
    from sejong_amd.benchmark import cached_measurement
    from sejong_amd.corpus import Corpus
    from sejong_amd.model import config
    rng = np.random.default_rng(2)
    (tmp_path / "v.txt").write_bytes(rng.integers(0, 256, 5000, dtype=np.uint8).tobytes())
    mc, tc = config("cfg2")
    tc.batch = 1
    m, _ = _model(mc, tc)
    try:
        rep = cached_measurement(m, Corpus.open(tmp_path), 16)
        print(f"[infer] {rep}")
        assert rep["prefill_tokens"] == 496 and rep["decode_tokens"] == 16
        assert rep["cached_vs_full_last_logits_max_abs_error"] <= TOL
        assert rep["decode_tokens_per_second"] > 0
    finally:
        m.close()


@pytest.mark.parametrize("graph", [False, True])
def test_inference_after_training_uses_updated_weights(graph):
    """A training step leaves the transposed weight mirror to the next
    forward, which rebuilds it beside its layers; inference after training
    must still see the updated weights: the trained model's cached decode
    and full logits equal those of a fresh model given its parameters."""
    from sejong_amd.benchmark import full_logits
    from sejong_amd.model import Model, byte_batch, config, init_params
    from sejong_amd.rng import Rng
    mc, tc = config("cfg2")
    mc.layers, tc.batch, tc.sequence = 2, 2, 128
    params = init_params(mc, std=0.02)
    ids, tg = byte_batch(Rng(9), tc.batch, tc.sequence)
    a = Model(mc, tc)
    b = Model(mc, tc)
    try:
        a.set_params(params)
        a.set_batch(ids, tg)
        a.use_graph(graph)
        for _ in range(3):
            a.train_step(1e-2)
        trained = a.get_params()
        assert np.any(trained != params)
        seq = np.random.default_rng(4).integers(0, 256, tc.sequence).astype(np.int32)
        ca = a.new_cache()
        got = [a.forward_cached(seq[:100], ca)] + [a.forward_cached(seq[p:p + 1], ca) for p in range(100, 104)]
        b.set_params(trained)
        cb = b.new_cache()
        ref = [b.forward_cached(seq[:100], cb)] + [b.forward_cached(seq[p:p + 1], cb) for p in range(100, 104)]
        for x, y in zip(got, ref):
            np.testing.assert_array_equal(x, y)
        a.train_step(1e-2)  # and the forward-only path after another step
        b.set_params(a.get_params())
        np.testing.assert_array_equal(full_logits(a, seq), full_logits(b, seq))
        ca.close(); cb.close()
    finally:
        a.close(); b.close()


def _hier_model(precision, P, T, seed=5):
    """A cfg3-family hierarchical model (encoder, global stack over patches,
    decoder; local window 96) with a non-zero global_bos row, so the first
    patch's context is not zero."""
    from sejong_amd.model import HierarchyConfig, Model, ModelConfig, TrainConfig, init_params
    mc = ModelConfig(width=512, layers=2, heads=8, kv_heads=2, ffn_width=1376, context=T, precision=precision,
                     hierarchy=HierarchyConfig(patch_size=P, encoder_width=256, encoder_layers=1, encoder_heads=4,
                                               encoder_ffn_width=768, decoder_width=256, decoder_layers=2,
                                               decoder_heads=4, decoder_ffn_width=768, local_window=96))
    tc = TrainConfig(sequence=T, batch=1)
    params = init_params(mc, std=0.02, seed=seed)
    m = Model(mc, tc)
    for name, (r, c), off in m.param_info():
        if name == "global_bos":
            params[off:off + r * c] = np.random.default_rng(seed).normal(0, 0.5, r * c).astype(np.float32)
    m.set_params(params)
    return m


def _chunk_plans(T, P):
    """Call sequences over one sequence of T bytes: token by token from an
    empty cache (every position; the first call is shorter than a patch);
    a first call shorter than a patch, then uneven chunks that end inside
    patches and cross several; a prefill with a partial last patch, then
    single bytes through several patches and longer chunks; the whole
    sequence at once."""
    def fill(plan):
        plan = list(plan)
        rest = T - sum(plan)
        while rest > 0:
            n = min(rest, 1 + (len(plan) * 7) % 23)
            plan.append(n)
            rest -= n
        return plan
    return [[1] * T,
            fill([P - 1, 1, 1, P + 2, 2 * P + 1, 1, 64 // P * P - 1, 2, 1]),
            fill([2 * P + 2] + [1] * (3 * P + 1) + [P + 3, 5 * P, 1]),
            [T]]


@pytest.mark.parametrize("precision,P,T", [("bf16", 4, 256), ("f32", 3, 128)])
def test_hierarchical_cached_vs_full(precision, P, T):
    """The hierarchical cached forward (HierarchyCache, hierarchical_prefill
    and the patch loop of hidden_cached, architecture.rs:395-452, 534-799)
    against the full forward's logits at the last byte of every call, for
    prefills shorter and longer than a patch, uneven chunks and decoding
    through several patches (the fp32 case with patch 3 ends on a partial
    patch); the cache reset between plans (HierarchyCache::reset) clears the
    patch state.  The reference's gate is 1e-4 (system_check.rs:48-51);
    the cached path pools a completed patch with the full forward's own
    kernel and runs every row through the same kernels, so the logits come
    out bit-identical."""
    from sejong_amd.benchmark import full_logits
    m = _hier_model(precision, P, T)
    try:
        ids = np.random.default_rng(T + P).integers(0, 256, T).astype(np.int32)
        full = full_logits(m, ids)
        cache = m.new_cache()
        for k, plan in enumerate(_chunk_plans(T, P)):
            cache.reset()
            pos, worst = 0, 0.0
            print(f"[infer] hierarchical {precision} P={P} T={T} plan {k}: {len(plan)} calls", flush=True)
            for n in plan:
                got = m.forward_cached(ids[pos:pos + n], cache)
                pos += n
                err = float(np.max(np.abs(got.astype(np.float64) - full[pos - 1])))
                assert err <= TOL, (k, pos, n, err)
                worst = max(worst, err)
            assert pos == T == cache.length
            print(f"[infer] hierarchical plan {k}: max abs error {worst:.3e}", flush=True)
        from sejong_amd import _native as N
        with pytest.raises(N.SejongError, match="context limit"):
            m.forward_cached(ids[:1], cache)
        cache.close()
    finally:
        m.close()


def test_cached_measurement_report_cfg3(tmp_path):
    """cached_measurement (benchmark.rs:113-171) on the cfg3 hierarchical
    model (1024 bytes, patches of 4): prefill of 1008 bytes (252 patches),
    then 16 bytes decoded one at a time through four patches; the error of
    the last byte's logits within the 1e-4 gate."""
    from sejong_amd.benchmark import cached_measurement
    from sejong_amd.corpus import Corpus
    from sejong_amd.model import config
    rng = np.random.default_rng(3)
    (tmp_path / "v.txt").write_bytes(rng.integers(0, 256, 5000, dtype=np.uint8).tobytes())
    mc, tc = config("cfg3")
    tc.batch = 1
    m, _ = _model(mc, tc)
    try:
        rep = cached_measurement(m, Corpus.open(tmp_path), 16)
        print(f"[infer] cfg3 {rep}", flush=True)
        assert rep["prefill_tokens"] == 1008 and rep["decode_tokens"] == 16
        assert rep["cached_vs_full_last_logits_max_abs_error"] <= TOL
        assert rep["decode_tokens_per_second"] > 0
    finally:
        m.close()
