"""Patch pool / broadcast of the hierarchical (cfg3) model and their
backwards against the oracle's restatement of the reference kernels
(oracle/hierarchy.py: fp32 sums in the reference's order): bit for bit, at
the cfg3 shape (8 sequences of 1024 bytes, encoder width 256, 4-byte
patches), a ragged last patch, a patch longer than the sequence and widths
that take the scalar path."""
import numpy as np
import pytest

from oracle import hierarchy as OH
from oracle import oracle as O
from tests.gpu_util import dev, empty, sync

pytestmark = pytest.mark.gpu
DT = {"f32": 0, "bf16": 4}

CASES = [(8, 1024, 256, 4, "bf16"), (8, 1024, 256, 4, "f32"), (3, 1022, 256, 4, "bf16"), (2, 5, 64, 8, "f32"),
         (2, 37, 100, 3, "f32"), (2, 37, 12, 3, "bf16"), (1, 64, 512, 1, "bf16")]


@pytest.mark.parametrize("B,T,d,P,dtype", CASES)
def test_patch_maps_bit_exact(B, T, d, P, dtype):
    from sejong_amd import _native as N
    N.load()
    api = N.api
    rng = np.random.default_rng(B * 1000 + T + d + P)
    NP = -(-T // P)
    x = O.round_to(rng.normal(size=(B * T, d)), dtype)
    X, Y = dev(x, dtype), empty(B * NP * d, dtype)
    api.sj_patch_pool(None, X.p, DT[dtype], B, T, d, P, Y.p)
    dy = rng.normal(size=(B * NP, d)).astype(np.float32).astype(np.float64)
    DY, DX = dev(dy), empty(B * T * d)
    api.sj_patch_pool_bwd(None, DY.p, B, T, d, P, DX.p)
    z = O.round_to(rng.normal(size=(B * NP, d)), dtype)
    bos = O.round_to(rng.normal(size=d), dtype)
    Z, BOS, YB = dev(z, dtype), dev(bos, dtype), empty(B * T * d, dtype)
    api.sj_patch_broadcast(None, Z.p, BOS.p, DT[dtype], B, T, d, P, YB.p)
    g = rng.normal(size=(B * T, d)).astype(np.float32).astype(np.float64)
    G, GX, GB = dev(g), empty(B * NP * d), empty(d)
    api.sj_patch_broadcast_bwd(None, G.p, B, T, d, P, GX.p, GB.p)
    sync()
    np.testing.assert_array_equal(Y.host(), OH.patch_pool(x, B, T, P, dtype).ravel())
    np.testing.assert_array_equal(DX.host(), OH.patch_pool_backward(dy, B, T, P).ravel())
    np.testing.assert_array_equal(YB.host(), OH.patch_broadcast(z, bos, B, T, P).ravel())
    ex, eb = OH.patch_broadcast_backward(g, B, T, P)
    np.testing.assert_array_equal(GX.host(), ex.ravel())
    np.testing.assert_array_equal(GB.host(), eb)
