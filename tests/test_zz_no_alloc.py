"""The allocation-free RMSNorm backward (sj_rmsnorm_bwd_p_noalloc) against
the workspace entry point sj_rmsnorm_bwd_p: bit-identical outputs on two
calls in a row, the second smaller than the first (the shared device array
keeps the first call's partials), and the capacity error past its maximum.

Collected last on purpose: a failure here cannot hide the other tests."""
import ctypes

import numpy as np
import pytest

from tests.gpu_util import dev, empty, rnd, sync, zeros

pytestmark = pytest.mark.gpu
cf = ctypes.c_float


@pytest.fixture(scope="module")
def api():
    from sejong_amd import _native as N
    N.load()
    return N.api


@pytest.fixture(scope="module")
def lib():
    from sejong_amd import _native as N
    return N.load()


def _run(api, lib, R, D, ldt, seed, noalloc):
    rng = np.random.default_rng(seed)
    x = rnd((R, D), "bf16", rng); w = rnd(D, "bf16", rng)
    dy = rng.normal(0, 1e-3, (R, D)).astype(np.float32)
    acc = rng.normal(0, 1e-3, (R, D)).astype(np.float32)
    X, W, DY, ACC = dev(x, "bf16"), dev(w, "bf16"), dev(dy), dev(acc)
    DX, DW = empty(R * D), empty(D)
    Hn, Ln = empty(R * D, "bf16"), empty(R * D, "bf16")
    Ht, Lt = zeros(D * ldt, "bf16"), zeros(D * ldt, "bf16")
    if noalloc:
        api.sj_rmsnorm_bwd_p_noalloc(None, X.p, W.p, DY.p, ACC.p, DX.p, DW.p, Hn.p, Ln.p, Ht.p, Lt.p, ldt, R, D,
                                     cf(1e-6))
    else:
        ws = empty(max(lib.sj_rmsnorm_bwd_p_workspace_bytes(R, D), 256), "u8")
        api.sj_rmsnorm_bwd_p(None, X.p, W.p, DY.p, ACC.p, DX.p, DW.p, Hn.p, Ln.p, Ht.p, Lt.p, ldt, R, D, cf(1e-6),
                             ws.p, ws.nbytes)
    sync()
    return [b.host() for b in (DX, DW, Hn, Ln, Ht, Lt)]


def test_noalloc_matches_workspace_entry_twice(api, lib):
    # first call at the cfg2 norm shape, the second smaller (fewer row groups
    # and columns): stale partials from the first call must not leak in
    for R, D, ldt, seed in [(4096, 384, 4096, 1), (1000, 256, 1000, 2)]:
        print(f"[no_alloc] rows {R} d {D}", flush=True)
        want = _run(api, lib, R, D, ldt, seed, noalloc=False)
        got = _run(api, lib, R, D, ldt, seed, noalloc=True)
        for name, a, b in zip(("dx", "dw", "dx_hi", "dx_lo", "dx_t_hi", "dx_t_lo"), got, want):
            np.testing.assert_array_equal(a, b, err_msg=f"{name} rows {R} d {D}")


def test_noalloc_allocates_no_device_memory(api, lib):
    """After a warm-up call (the module's code object loaded, the shared
    array's address resolved), further calls leave the device's free memory
    unchanged: the entry point allocates nothing."""
    R, D, ldt = 4096, 384, 4096
    rng = np.random.default_rng(3)
    X, W = dev(rnd((R, D), "bf16", rng), "bf16"), dev(rnd(D, "bf16", rng), "bf16")
    DY, ACC = dev(rng.normal(0, 1e-3, (R, D)).astype(np.float32)), dev(np.zeros((R, D), np.float32))
    DX, DW = empty(R * D), empty(D)
    Hn, Ln, Ht, Lt = empty(R * D, "bf16"), empty(R * D, "bf16"), empty(D * ldt, "bf16"), empty(D * ldt, "bf16")

    def call(rows):  # the wrapped entry point raises on a non-zero status
        api.sj_rmsnorm_bwd_p_noalloc(None, X.p, W.p, DY.p, ACC.p, DX.p, DW.p, Hn.p, Ln.p, Ht.p, Lt.p, ldt, rows, D,
                                     cf(1e-6))
        sync()

    def free():
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        api.sj_memory_info(ctypes.byref(f), ctypes.byref(t))
        return f.value

    call(R)
    before = free()
    for rows in (R, 1000, R):
        call(rows)
    assert free() == before


def test_noalloc_rejects_beyond_maximum(lib):
    from sejong_amd import _native as N
    cap = N.load().sj_rmsnorm_bwd_p_workspace_bytes(16 * 1025, 1024)
    assert cap > 4 << 20
    st = lib.sj_rmsnorm_bwd_p_noalloc(None, None, None, None, None, None, None, None, None, None, None, 0,
                                      16 * 1025, 1024, cf(1e-6))
    assert st == 2 and b"no allocation" in lib.sj_last_error()
