"""End-to-end parity of the native training step (sj_model_*) against the
FP64 oracle: loss, every parameter gradient (reference layout), the AdamW
update, determinism and hipGraph replay.

Protocol.  fp32 storage (cfg1) is compared end to end.  With bf16 storage
an end-to-end comparison is ill-conditioned: the oracle itself moves its
gradients by ~0.6% (worst tensor) when the parameters change by 1e-7,
because near-tie bf16 roundings of the activations flip (measured on the
CPU at the cfg2 shape, 2 layers).  So, as the reference's own FP64 checks do
(they condition on the stored O(F16) and LSE(F32)), the oracle consumes the
device's stored operands: every forward op is re-derived from the stored
inputs of that op (within one storage ulp per rounding), and the whole
backward is recomputed in FP64 from the stored activations; loss and every
parameter gradient must then agree within 1e-3 relative (the gate).
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import rel

pytestmark = pytest.mark.gpu

GRAD_TOL = 1e-3  # relative, per parameter tensor (north-star gate)


def _oracle_cfg(mc, tc):
    return dict(d=mc.width, layers=mc.layers, hq=mc.heads, hk=mc.kv, ffn=mc.ffn_width, T=tc.sequence, B=tc.batch,
                eps=mc.norm_epsilon, theta=mc.rope_theta)


def _per_tensor_rel(info, got, ref):
    out = {}
    for name, (r, c), off in info:
        n = r * c
        g, e = got[off:off + n].astype(np.float64), ref[off:off + n]
        den = np.linalg.norm(e)
        out[name] = np.linalg.norm(g - e) / den if den > 0 else np.linalg.norm(g)
    return out


def _device_step(mc, tc, seed=0):
    from sejong_amd.model import Model, byte_batch, init_params
    from sejong_amd.rng import Rng
    params = init_params(mc, std=0.02, seed=42 + seed)
    ids, tg = byte_batch(Rng(123 + seed), tc.batch, tc.sequence)
    model = Model(mc, tc)
    model.set_params(params)
    model.set_batch(ids, tg)
    model.forward_backward()
    loss, _ = model.read_loss()
    return model, params, ids, tg, loss, model.get_grads()


def _split_acts(cfg, acts):
    out, off = {}, 0
    for name, layer, size in O.acts_layout(cfg):
        out[(name, layer)] = acts[off:off + size]
        off += size
    return out


def _params_by_name(info, params):
    return {name: params[off:off + r * c].astype(np.float64).reshape((r, c) if r > 1 else (c,))
            for name, (r, c), off in info}


def _ulp_check(got, ref, scale, ulps, what, terms=None):
    """|got - ref| <= ulps * 2^-7 * scale + 2^-16 * terms elementwise (bf16
    storage; `terms` = sum of |products| behind the element, for the fp32
    accumulation error of results that cancel)."""
    err = np.abs(got - ref)
    tol = ulps * 2.0 ** -7 * np.maximum(scale, 1e-30) + (0 if terms is None else 2.0 ** -16 * terms)
    bad = err > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} beyond {ulps} ulp: {got[bad][:3]} vs {ref[bad][:3]}"


def _check_forward_conditioned(cfg, info, params, ids, acts):
    """Re-derive every stored forward activation from the stored inputs."""
    P = _params_by_name(info, params)
    Pc = {k: O.round_to(v, "bf16") if k != "output" else v for k, v in P.items()}
    A = _split_acts(cfg, acts)
    M, d, L, T = cfg["T"] * cfg["B"], cfg["d"], cfg["layers"], cfg["T"]
    hq, hk, F = cfg["hq"], cfg["hk"], cfg["ffn"]
    Dh = d // hq; J = Dh * hk
    eps = cfg["eps"]
    r2 = lambda k, l, n: A[(k, l)].reshape(M, n)
    np.testing.assert_array_equal(r2("x", 0, d), Pc["embedding"][ids])
    for l in range(L):
        p = f"layers.{l}."
        x, z = r2("x", l, d), r2("z", l, d)
        ref = O.rmsnorm_fwd(x, Pc[p + "attention_norm"], eps)
        _ulp_check(z, ref, np.abs(ref), 1, f"z[{l}]")
        az = np.abs(z)
        q = O.round_to(z @ Pc[p + "query"], "bf16"); k = O.round_to(z @ Pc[p + "key"], "bf16")
        rq = O.rope(q, T, hq, Dh); rk = O.rope(k, T, hk, Dh)
        pm = lambda a, H: np.repeat(np.abs(a).reshape(M, H, Dh // 2, 2).max(-1), 2, -1).reshape(M, H * Dh)
        _ulp_check(r2("qr", l, d), rq, 2 * pm(q, hq), 1, f"q[{l}]", terms=pm(az @ np.abs(Pc[p + "query"]), hq))
        _ulp_check(r2("kr", l, J), rk, 2 * pm(k, hk), 1, f"k[{l}]", terms=pm(az @ np.abs(Pc[p + "key"]), hk))
        vref = z @ Pc[p + "value"]
        _ulp_check(r2("v", l, J), vref, np.abs(vref), 1, f"v[{l}]", terms=az @ np.abs(Pc[p + "value"]))
        qr_, kr_, v_ = r2("qr", l, d), r2("kr", l, J), r2("v", l, J)
        o_ref, lse_ref = O.attention_fwd(qr_, kr_, v_, cfg["B"], T, hq, hk, Dh)
        o_abs, _ = O.attention_fwd(qr_, kr_, np.abs(v_), cfg["B"], T, hq, hk, Dh)
        _ulp_check(r2("o", l, d), o_ref, np.abs(o_ref), 1, f"o[{l}]", terms=2 * o_abs)
        assert rel(A[("lse", l)], lse_ref) < 1e-5
        o = r2("o", l, d)
        a = o @ Pc[p + "attention_output"]
        x1 = r2("x1", l, d)
        _ulp_check(x1, x + a, np.abs(a) + np.abs(x1), 1, f"x1[{l}]", terms=np.abs(o) @ np.abs(Pc[p + "attention_output"]))
        z2 = r2("z2", l, d)
        ref = O.rmsnorm_fwd(x1, Pc[p + "ffn_norm"], eps)
        _ulp_check(z2, ref, np.abs(ref), 1, f"z2[{l}]")
        gref, uref = z2 @ Pc[p + "gate"], z2 @ Pc[p + "up"]
        g, u, h = r2("g", l, F), r2("u", l, F), r2("h", l, F)
        az2 = np.abs(z2)
        _ulp_check(g, gref, np.abs(gref), 1, f"g[{l}]", terms=az2 @ np.abs(Pc[p + "gate"]))
        _ulp_check(u, uref, np.abs(uref), 1, f"u[{l}]", terms=az2 @ np.abs(Pc[p + "up"]))
        href = O.swiglu_fwd(g, u)
        _ulp_check(h, href, np.abs(href), 1, f"h[{l}]")
        f = h @ Pc[p + "down"]
        xn = r2("x", l + 1, d) if l + 1 < L else A[("xL", -1)].reshape(M, d)
        _ulp_check(xn, x1 + f, np.abs(f) + np.abs(xn), 1, f"x[{l + 1}]", terms=np.abs(h) @ np.abs(Pc[p + "down"]))
    xl, hn = A[("xL", -1)].reshape(M, d), A[("hn", -1)].reshape(M, d)
    ref = O.rmsnorm_fwd(xl, Pc["final_norm"], eps)
    _ulp_check(hn, ref, np.abs(ref), 1, "hn")
    assert rel(A[("logits", -1)], (hn @ P["output"]).ravel()) < 1e-5


def _conditioned_parity(mc, tc, seed=0):
    model, params, ids, tg, loss, grads = _device_step(mc, tc, seed)
    try:
        info = model.param_info()
        cfg = _oracle_cfg(mc, tc)
        acts = np.empty(model.activation_count(), np.float32)
        model.export_activations(acts)
        acts = acts.astype(np.float64)
        assert acts.size == O.model_acts_count(cfg)
        _check_forward_conditioned(cfg, info, params, ids, acts)
        lref, gref, _ = O.model_backward(cfg, params.astype(np.float64), acts, ids, tg, dtype=mc.precision)
        rels = _per_tensor_rel(info, grads, gref)
        worst = max(rels.items(), key=lambda kv: kv[1])
        print(f"[parity] conditioned: loss {loss:.8f} vs {lref:.8f}; worst grad rel {worst}", flush=True)
        assert abs(loss - lref) < 1e-6 * abs(lref)
        bad = {k: v for k, v in rels.items() if not v < GRAD_TOL}
        assert not bad, bad
        # unconditioned end to end: the bf16 noise floor (see module doc)
        lu, gu, _, _ = O.model_fwd_bwd(cfg, params.astype(np.float64), ids, tg, dtype=mc.precision)
        ru = _per_tensor_rel(info, grads, gu)
        wu = max(ru.values())
        print(f"[parity] end-to-end: loss {loss:.7f} vs {lu:.7f}; worst grad rel {wu:.3e}", flush=True)
        assert abs(loss - lu) < 1e-4 * abs(lu) and wu < 5e-2
        return rels
    finally:
        model.close()


def test_cfg1_fp32_end_to_end():
    from sejong_amd.model import config
    mc, tc = config("cfg1")
    model, params, ids, tg, loss, grads = _device_step(mc, tc)
    try:
        lref, gref, _, _ = O.model_fwd_bwd(_oracle_cfg(mc, tc), params.astype(np.float64), ids, tg, dtype="f32")
        rels = _per_tensor_rel(model.param_info(), grads, gref)
        worst = max(rels.items(), key=lambda kv: kv[1])
        print(f"[parity] cfg1: loss {loss:.8f} vs {lref:.8f}; worst grad rel {worst}", flush=True)
        assert abs(loss - lref) < 1e-6 * abs(lref)
        assert worst[1] < GRAD_TOL
    finally:
        model.close()


@pytest.mark.parametrize("name", ["cfg2-2layer", "cfg2", "wide-ffn"])
def test_bf16_conditioned_parity(name):
    from sejong_amd.model import config
    mc, tc = config("cfg2")
    if name == "cfg2-2layer":
        mc.layers, tc.batch, tc.sequence = 2, 2, 256
    if name == "wide-ffn":
        # M*F = 4096 * 2304 > 8 Mi: the down-projection dW is enqueued after
        # the SwiGLU planes are written (the other stream order of the step)
        mc.layers, mc.ffn_width = 2, 2304
    print(f"[parity] {name}: d={mc.width} L={mc.layers} B={tc.batch} T={tc.sequence} {mc.precision}", flush=True)
    _conditioned_parity(mc, tc)


def test_adamw_step_matches_oracle_update():
    """train_step = forward/backward (bit-identical to the one read back) +
    FP64 norm, clip and AdamW; compared with the oracle's AdamW on the
    device gradients (Adam::update, crates/sejong-train/src/lib.rs:199-238)."""
    from sejong_amd.model import config
    mc, tc = config("cfg2")
    mc.layers, tc.batch, tc.sequence = 2, 2, 128
    model, params, ids, tg, loss_dev, grads = _device_step(mc, tc, seed=1)
    try:
        model.train_step(tc.learning_rate)
        loss2, norm = model.read_loss()
        assert loss2 == loss_dev  # deterministic recompute
        new = model.get_params()
        m, v, step = model.get_adam_state()
        assert step == 1
        g = grads.astype(np.float64)
        gn = math.sqrt(O.sum_squares(g))
        assert abs(norm - gn) < 1e-9 * gn
        clip = tc.clip_norm / gn if gn > tc.clip_norm else 1.0
        scale = float(np.float32(clip))
        ib1 = float(np.float32(1) / (np.float32(1) - np.float32(tc.beta1) ** np.float32(1)))
        ib2 = float(np.float32(1) / (np.float32(1) - np.float32(tc.beta2) ** np.float32(1)))
        decay = np.zeros(params.size)
        for name, (r, c), off in model.param_info():
            if r > 1:  # matrices decay (p.value.shape.len() > 1)
                decay[off:off + r * c] = 1.0
        lr32 = float(np.float32(tc.learning_rate))
        ref_w = np.empty(params.size)
        for dflag in (0.0, 1.0):
            sel = decay == dflag
            ref_w[sel] = O.adamw(params[sel].astype(np.float64), g[sel], np.zeros(sel.sum()), np.zeros(sel.sum()),
                                 lr32, 0.9, 0.95, 0.0, dflag * float(np.float32(tc.weight_decay)), ib1, ib2, scale)[0]
        assert np.max(np.abs(new - ref_w)) < 2e-7
        assert np.max(np.abs(m - (1 - np.float32(0.9)) * g * scale)) < 1e-9 + 1e-6 * np.abs(m).max()
    finally:
        model.close()


def test_graph_replay_equals_eager_and_is_deterministic():
    from sejong_amd.model import Model, byte_batch, config, init_params
    from sejong_amd.rng import Rng
    mc, tc = config("cfg2")
    mc.layers, tc.batch, tc.sequence = 2, 2, 128
    params = init_params(mc, std=0.02)
    ids, tg = byte_batch(Rng(5), tc.batch, tc.sequence)
    out = []
    for graph in (False, True, True):
        model = Model(mc, tc)
        model.set_params(params)
        model.set_batch(ids, tg)
        model.use_graph(graph)
        losses = []
        for i in range(4):
            model.train_step(1e-3)
            losses.append(model.read_loss()[0])
        out.append((model.get_params(), losses))
        model.close()
    np.testing.assert_array_equal(out[0][0], out[1][0])
    np.testing.assert_array_equal(out[1][0], out[2][0])
    assert out[0][1] == out[1][1]
    assert out[0][1][-1] < out[0][1][0]  # the loss moves down on a fixed batch


def test_graph_replay_equals_eager_at_bench_configuration():
    """The step bench.py times, at its configuration (full cfg2: 6 layers,
    B 8 x T 512, the dW products on the second stream, the gradient planes
    reused by layer parity, the attention backward's plan with cut walks):
    two AdamW steps replayed from the captured graph leave the parameters,
    gradients, Adam moments and losses bit-identical to two eager steps."""
    from sejong_amd.model import Model, byte_batch, config, init_params
    from sejong_amd.rng import Rng
    mc, tc = config("cfg2")
    params = init_params(mc, std=0.02)
    ids, tg = byte_batch(Rng(123), tc.batch, tc.sequence)
    out = []
    for graph in (False, True):
        model = Model(mc, tc)
        try:
            model.set_params(params)
            model.set_batch(ids, tg)
            model.use_graph(graph)
            losses = []
            for _ in range(2):
                model.train_step(tc.learning_rate)
                losses.append(model.read_loss())
            m, v, step = model.get_adam_state()
            out.append((model.get_params(), model.get_grads(), m, v, step, losses))
            print(f"[graph] cfg2 graph={graph}: losses {losses}", flush=True)
        finally:
            model.close()
    for name, a, b in zip(("params", "grads", "m", "v"), out[0][:4], out[1][:4]):
        np.testing.assert_array_equal(a, b, err_msg=name)
    assert out[0][4] == out[1][4] == 2
    assert out[0][5] == out[1][5]


def test_profiled_steps_equal_plain_steps_and_time_their_gemm_kernels():
    """Per-op profiling in kernel-timing mode (sj_model_profile 3) runs the
    step on one stream and launches each GEMM op's kernel with events at its
    own start and end: the
    parameters after two profiled steps equal those of two plain steps
    bit for bit, every GEMM op reports a "#kernel" aggregate no longer than
    the op and names its GEMM kernel (the attention ops: their attention
    kernel), other ops name none."""
    from sejong_amd.model import Model, byte_batch, config, init_params
    from sejong_amd.rng import Rng
    mc, tc = config("cfg2")
    mc.layers, tc.batch, tc.sequence = 2, 2, 128
    params = init_params(mc, std=0.02)
    ids, tg = byte_batch(Rng(7), tc.batch, tc.sequence)
    out = []
    for prof in (False, True):
        model = Model(mc, tc)
        try:
            model.set_params(params)
            model.set_batch(ids, tg)
            model.profile(prof, kernels=True)
            for _ in range(2):
                model.train_step(1e-3)
            if prof:
                agg = model.profile_collect()
                kern = dict(model.profile_kernels)
                model.profile(False)
            out.append(model.get_params())
        finally:
            model.close()
    np.testing.assert_array_equal(out[0], out[1])
    gemm_ops = ["qkv_rope", "attn_out_residual", "gate_up_swiglu", "down_residual", "qkv_dx", "qkv_dw",
                "attn_out_dx", "attn_out_dw", "gate_up_dx", "gate_up_dw", "down_dx_swiglu", "down_dw"]
    for op in gemm_ops:
        assert op in agg and op + "#kernel" in agg, op
        ms, calls = agg[op]
        kms, kcalls = agg[op + "#kernel"]
        assert calls == kcalls == 2 * mc.layers, (op, calls, kcalls)
        assert 0 < kms <= ms, (op, kms, ms)
        assert kern[op].startswith(("k_gemm_fast<", "k_gemm_kw<")) and kern[op] == kern[op + "#kernel"], (op, kern[op])
    # the attention kernels time themselves the same way; other ops name no kernel
    for op, name in (("attention_fwd", "k_attn2_fwd<3>"), ("attention_bwd_dq_dkv", "k_attn2_bwd_g<3>")):
        assert op in agg and op + "#kernel" in agg and kern[op] == name, (op, kern.get(op))
        assert 0 < agg[op + "#kernel"][0] <= agg[op][0], op
    for op in ("rmsnorm", "adamw"):
        assert op in agg and kern[op] == "", (op, kern.get(op))


def test_gradient_norm_from_producer_partials():
    """The bf16 step sums the squared gradient norm from FP64 partials its
    gradient producers write (split-K dW reduce, norm-weight reduce,
    embedding backward) instead of a pass over the arena: the norm the step
    reports equals the FP64 norm of the gradients it left, at the full cfg2
    shape (every dW product split) and at a 2-layer cut, eager and replayed."""
    from sejong_amd.model import Model, byte_batch, config, init_params
    from sejong_amd.rng import Rng
    for layers, batch in ((6, 8), (2, 2)):
        mc, tc = config("cfg2")
        mc.layers, tc.batch = layers, batch
        params = init_params(mc, std=0.02)
        ids, tg = byte_batch(Rng(3), tc.batch, tc.sequence)
        for graph in (False, True):
            model = Model(mc, tc)
            try:
                model.set_params(params)
                model.set_batch(ids, tg)
                model.use_graph(graph)
                for _ in range(2):
                    model.train_step(1e-3)
                _, norm = model.read_loss()
                g = model.get_grads().astype(np.float64)
                ref = math.sqrt(float(np.dot(g, g)))
                assert abs(norm - ref) <= 1e-12 * ref, (layers, graph, norm, ref)
                _, slots = model.buffer("grad_sq_slots")
                assert slots > 0, (layers, graph)  # the producers' partials were summed
            finally:
                model.close()
