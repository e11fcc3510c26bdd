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
