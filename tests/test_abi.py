"""CPU checks of the C ABI library and the host-side logic (no GPU calls)."""
import math
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sejong_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(sj_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_parses():
    names = declared_functions()
    assert "sj_gemm" in names and "sj_model_train_step" in names and len(names) > 30


def test_library_exports_every_declared_symbol():
    from sejong_amd import _native as N
    lib = N.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_header():
    from sejong_amd import _native as N
    assert set(declared_functions()) == set(N.SIGNATURES)


def test_status_strings_without_gpu():
    from sejong_amd import _native as N
    lib = N.load()
    assert lib.sj_status_string(0) == b"ok"
    assert b"nonfinite" in lib.sj_status_string(5)


def test_shape_errors_are_reported_before_launch():
    # argument validation runs on the host: no device is touched
    from sejong_amd import _native as N
    lib = N.load()
    st = lib.sj_gemm(None, 0, 0, 4, 4, 4, None, N.SJ_F64, 4, None, N.SJ_BF16, 4, None, N.SJ_F32, 4, 0, None, 0)
    assert st == 1 and b"dtype" in lib.sj_last_error()
    st = lib.sj_gemm(None, 0, 0, 4, 4, 8, None, N.SJ_BF16, 4, None, N.SJ_BF16, 4, None, N.SJ_F32, 4, 0, None, 0)
    assert st == 1 and b"inner dimension" in lib.sj_last_error()
    st = lib.sj_attention_fwd(None, None, 64, None, 64, None, 64, None, 64, None, N.SJ_BF16, 1, 8, 3, 2, 64, 0)
    assert st == 1


def test_product_rng_matches_oracle_rng(oracle):
    from sejong_amd.rng import Rng
    a, b = Rng(42), oracle.Rng(42)
    assert [int(x) for x in a.next_block(10)] == [b.next_u64() for _ in range(10)]
    a, b = Rng(5), oracle.Rng(5)
    assert [a.index(1000) for _ in range(20)] == [b.index(1000) for _ in range(20)]
    np.testing.assert_allclose(Rng(9).normal(1000, 0.02), oracle.Rng(9).normal_fill(1000, 0.02), rtol=1e-15)


def test_layout_matches_baseline_count():
    from sejong_amd.model import config, param_count, layout
    mc, _ = config("cfg2")
    assert param_count(mc) == 9_639_552  # BASELINE.md cfg2 AdamW line
    names = [n for n, _, _ in layout(mc)]
    assert names[0] == "embedding" and names[-1] == "output" and names[1] == "layers.0.attention_norm"
    mc1, _ = config("cfg1")
    from oracle import oracle as O
    assert param_count(mc1) == O.model_param_count(128, 1, 4, 2, 384)


def test_byte_batch_is_shifted():
    from sejong_amd.model import byte_batch
    from sejong_amd.rng import Rng
    ids, tg = byte_batch(Rng(123), 3, 16)
    assert ids.shape == (48,) and ids.max() < 256 and ids.min() >= 0
    np.testing.assert_array_equal(ids.reshape(3, 16)[:, 1:], tg.reshape(3, 16)[:, :-1])


def test_init_params_std_and_norms():
    from sejong_amd.model import config, init_params, layout
    mc, _ = config("cfg1")
    p = init_params(mc, std=0.02)
    off = 0
    for name, shape, norm in layout(mc):
        n = math.prod(shape)
        seg = p[off:off + n]
        if norm:
            assert np.all(seg == 1.0)
        elif n > 10000:
            assert abs(seg.std() - 0.02) < 2e-3
        off += n


def test_pvjp_host_cost_model_matches_oracle():
    """sj_pvjp_budget / sj_pvjp_selects_compression / the basis tolerance
    are host code (no GPU): bit-exact against the oracle's integer
    restatement of parameter_vjp.rs:85-130, 214-220 over a grid of shapes."""
    import ctypes
    from oracle import pvjp
    from sejong_amd import _native as N
    lib = N.load()
    L = ctypes.c_long
    for rank in (1, 8, 16, 33, 64):
        for frac in (0.05, 0.1, 0.4, 1.0):
            for br in (16, 32):
                for n, a, b, donor, uses in ((16384, 1024, 1024, 5504, 3), (16384, 1024, 5504, 5504, 2),
                                             (16384, 2752, 1024, 1024, 1), (67, 71, 97, 97, 2), (900, 1024, 64, 64, 2),
                                             (4096, 384, 640, 1024, 3)):
                    r, bl, s = L(), L(), L()
                    assert lib.sj_pvjp_budget(rank, frac, br, n, a, donor, ctypes.byref(r), ctypes.byref(bl),
                                              ctypes.byref(s)) == 0
                    assert (r.value, bl.value, s.value) == pvjp.budget(rank, frac, br, n, a, donor)
                    got = lib.sj_pvjp_selects_compression(rank, frac, br, n, a, b, donor, uses)
                    assert bool(got) == pvjp.selects_compression(rank, frac, br, n, a, b, donor, uses)
    for rows, rank in ((67, 33), (16384, 16), (10 ** 8, 64)):
        assert lib.sj_pvjp_basis_tolerance(rows, rank) == np.float32(pvjp.basis_tolerance(rows, rank))


def test_noalloc_rejects_oversize_before_any_device_call():
    # the capacity check runs on the host before the device is touched
    import ctypes

    from sejong_amd import _native as N
    lib = N.load()
    st = lib.sj_rmsnorm_bwd_p_noalloc(None, None, None, None, None, None, None, None, None, None, None, 0,
                                      16 * 1025, 1024, ctypes.c_float(1e-6))
    assert st == 2 and b"SJ_RMSNORM_BWD_NOALLOC_MAX_BYTES" in lib.sj_last_error()


def _attention_plan(lib, t, window, pairs=16, cus=256):
    import ctypes
    seg = np.zeros(256, np.uint32)
    ncut = ctypes.c_int(-1)
    n = lib.sj_attention_bwd_plan(t, window, pairs, cus, seg.ctypes.data, seg.size, ctypes.byref(ncut))
    pieces = []
    for x in (int(v) for v in seg[:max(n, 0)]):
        assert x >> 31
        pieces.append(dict(block=x & 63, first=(x >> 6) & 63, last=(x >> 12) & 63, role=(x >> 18) & 1,
                           cut=((x >> 19) & 255) - 1, part=(x >> 27) & 3, nparts=((x >> 29) & 3) + 1))
    return n, ncut.value, pieces


def _piece_us(p):
    """Modelled workgroup time of a piece (the planner's per-walk start and
    per-block costs, microseconds, and a cut part's meeting)."""
    n = p["last"] - p["first"] + 1
    return (5.0 + 1.85 * n if p["role"] == 0 else 6.6 + 2.9 * n) + (5.0 if p["cut"] >= 0 else 0.0)


def _dispatch_finish(pieces, pairs, cus):
    """Finish time of the launch's dispatch: pieces in order, each for every
    pair, to the CU free first (the planner's model, restated)."""
    import heapq
    free = [0.0] * cus
    end = 0.0
    for p in pieces:
        c = _piece_us(p)
        for _ in range(pairs):
            t = heapq.heappop(free) + c
            end = max(end, t)
            heapq.heappush(free, t)
    return end


@pytest.mark.parametrize("t,window,pairs", [(64, 0, 16), (128, 0, 16), (256, 0, 4), (320, 100, 1), (256, 128, 4),
                                            (512, 0, 16), (512, 300, 16), (512, 64, 16), (1024, 0, 3),
                                            (1024, 200, 8), (2048, 0, 2), (2048, 1000, 2), (512, 0, 64)])
def test_attention_backward_pieces_cover_every_walk_once(t, window, pairs):
    """The grouped attention backward's pieces (sj_attention_bwd_plan): every
    causal walk of both roles (dQ of query block qb over its visible key
    blocks, dK | dV of key block kb over the query blocks that see it, the
    walks of the per-block kernels) is covered exactly once, by a whole piece
    or by two parts that meet end to end, with distinct cut indices below
    ncut <= t/64 (the workspace holds that many pairs of sums); pieces come
    costliest first; and the chosen cuts finish the modelled dispatch no
    later than no cuts at all (earlier at the cfg2 shape, where the longest
    dK | dV walks are cut)."""
    from sejong_amd import _native as N
    lib = N.load()
    nb_blocks = t // 64
    W = window if window < t else 0
    n, ncut, pieces = _attention_plan(lib, t, window, pairs)
    assert 2 * nb_blocks <= n <= 4 * nb_blocks and 0 <= ncut <= nb_blocks
    walks = {}
    for i in range(nb_blocks):
        kb0 = (i * 64 - W + 1) // 64 if W > 0 and i * 64 - W + 1 > 0 else 0
        nqb = min(nb_blocks, (i * 64 + 63 + W - 1) // 64 + 1) if W > 0 else nb_blocks
        walks[(0, i)] = (kb0, i)
        walks[(1, i)] = (i, nqb - 1)
    # brute-force check of the walk bounds: the blocks holding a visible pair
    for (role, i), (lo, hi) in walks.items():
        vis = []
        for o in range(nb_blocks):
            qb, kb = (i, o) if role == 0 else (o, i)
            pairs_ = [(q, k) for q in range(qb * 64, qb * 64 + 64) for k in range(kb * 64, kb * 64 + 64, 7)]
            pairs_ += [(q, kb * 64 + 63) for q in range(qb * 64, qb * 64 + 64)]
            if any(k <= q and (W == 0 or k > q - W) for q, k in pairs_):
                vis.append(o)
        assert vis == list(range(lo, hi + 1)), (role, i, vis, lo, hi)
    covered = {k: [] for k in walks}
    cuts = {}
    for p in pieces:
        covered[(p["role"], p["block"])].append((p["first"], p["last"], p["part"]))
        if p["cut"] >= 0:
            assert p["cut"] < ncut
            cuts.setdefault(p["cut"], []).append((p["role"], p["block"], p["part"], p["nparts"]))
        else:
            assert p["part"] == 0 and p["nparts"] == 1
    for k, (lo, hi) in walks.items():
        parts = sorted(covered[k])
        assert parts[0][0] == lo and parts[-1][1] == hi and len(parts) <= 4, (k, parts)
        for (a0, a1, ap), (b0, b1, bp) in zip(parts, parts[1:]):
            assert b0 == a1 + 1 and bp == ap + 1, (k, parts)  # parts in walk order
        assert all(a0 <= a1 for a0, a1, _ in parts)
    assert sorted(cuts) == list(range(ncut))
    slots = 0
    for c, ps in cuts.items():
        n = ps[0][3]
        assert 2 <= n <= 4 and len(ps) == n and len({p[:2] for p in ps}) == 1, (c, ps)
        assert sorted(p[2] for p in ps) == list(range(n)) and all(p[3] == n for p in ps), (c, ps)
        slots += n
    assert slots <= 2 * nb_blocks  # the part sums fit the workspace
    assert all(_piece_us(x) >= _piece_us(y) - 1e-12 for x, y in zip(pieces, pieces[1:]))
    whole = sorted(({"role": r, "block": b, "first": lo, "last": hi, "cut": -1} for (r, b), (lo, hi) in walks.items()),
                   key=lambda p: -_piece_us(p))
    assert _dispatch_finish(pieces, pairs, 256) <= _dispatch_finish(whole, pairs, 256) + 1e-9
    if (t, window, pairs) == (512, 0, 16):  # cfg2: the longest dK | dV walks cut, none of dQ
        assert ncut >= 4 and all(p["role"] == 1 for p in pieces if p["cut"] >= 0)
        assert _dispatch_finish(pieces, pairs, 256) < 0.85 * _dispatch_finish(whole, pairs, 256)


@pytest.mark.parametrize("B,T,HQ,HK", [(8, 512, 6, 2), (1, 1024, 3, 1), (2, 256, 6, 2), (16, 1024, 12, 4)])
def test_attention_backward_workspace_accounting(B, T, HQ, HK):
    """The grouped attention backward's workspace (no device needed): the
    part sums of every cut walk of every (KV head, sequence) pair fit the
    partial region (12288 floats per part: 16 per thread of the 768-thread
    workgroup), and the meeting counters (64 words per pair, cut index
    pair * 64 + cut) sit past it, 256-byte aligned, in the last
    sj_attention_bwd_tt_counter_bytes bytes, which grow with the pairs so
    that no two pairs, and no two workspaces, share a counter."""
    from sejong_amd import _native as N
    lib = N.load()
    Dh = 64
    pairs = B * HK
    cnt = lib.sj_attention_bwd_tt_counter_bytes(B, HK)
    total = lib.sj_attention_bwd_tt_workspace_bytes(B, T, HQ, HK, Dh)
    assert cnt == 4 * 64 * pairs
    partial = 4 * (HQ // HK) * B * T * 2 * HK * Dh
    assert total == (partial + 255) // 256 * 256 + cnt
    n, ncut, pieces = _attention_plan(lib, T, 0, pairs)
    assert n > 0 and 0 <= ncut <= 64
    slots = sum(p["nparts"] for p in pieces if p["cut"] >= 0 and p["part"] == 0)
    if HQ == 3 * HK:  # the grouped launch: part sums of 12288 floats
        assert pairs * slots * 12288 * 4 <= partial


def test_pvjp_library_decisions_on_reference_production_shapes():
    """The library's host decision function (sj_pvjp_selects_compression)
    on every group the reference's production configuration forms (its
    recorded 44 compressed / 126 dense matrices: tests/test_oracle.py), with
    the retain loop's member counts: the same verdict as the oracle for the
    global q|k|v (512 patches x 512), the local q|k|v and gate|up (4096 bytes
    x 128) and the single-use and expert products (rank 16, residual 0.25,
    32-row blocks)."""
    from oracle import pvjp
    from sejong_amd import _native as N
    lib = N.load()
    cases = [  # n, a, b, donor, uses
        (512, 512, 512, 512, 3), (512, 512, 256, 512, 3),                 # global q, k / v
        (4096, 128, 128, 128, 3), (4096, 128, 384, 384, 2),               # local q|k|v, gate|up
        (4096, 128, 128, 128, 1), (4096, 384, 128, 128, 1),               # attention_output, down
        (512, 512, 4, 4, 1), (512, 128, 512, 512, 1), (4096, 512, 257, 257, 1),  # router, glue, head
        (256, 512, 384, 384, 2), (512, 512, 384, 384, 2)]                 # an expert's gate|up
    for n, a, b, donor, uses in cases:
        want = pvjp.selects_compression(16, 0.25, 32, n, a, b, donor, uses)
        assert bool(lib.sj_pvjp_selects_compression(16, 0.25, 32, n, a, b, donor, uses)) == want, (n, a, b, uses)
