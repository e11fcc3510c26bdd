"""Device-memory helpers for the GPU parity tests (torch is only the
allocator; every computation under test runs in libsejong_hip.so)."""
import ctypes

import numpy as np

from oracle import oracle as O


def torch():
    import torch as t
    return t


def dev(x, dtype="f32"):
    """Upload float64/float32 numpy values as an f32 / bf16 / i32 device tensor.
    bf16 inputs must already be bf16-representable (use O.round_to)."""
    t = torch()
    a = np.asarray(x)
    if dtype == "i32":
        return t.tensor(a.astype(np.int32), device="cuda")
    ten = t.tensor(a.astype(np.float32), device="cuda")
    return ten.to(t.bfloat16) if dtype == "bf16" else ten


def host(t_):
    return t_.float().cpu().numpy().astype(np.float64)


def p(t_):
    return ctypes.c_void_p(t_.data_ptr())


def sync():
    torch().cuda.synchronize()


def rnd(shape, dtype, rng, std=1.0):
    """Random values already rounded to the storage dtype."""
    return O.round_to(rng.normal(0, std, shape), dtype)


def rel(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    n = np.linalg.norm(b)
    return np.linalg.norm(a - b) / (n if n > 0 else 1.0)


def assert_stored_close(got, ref, dtype, what=""):
    """`got` was stored in `dtype`; `ref` is the FP64 value before that
    store.  Each element must be within one storage ulp of ref (the two sides
    may round a near-tie differently), and the tensor as a whole within the
    storage rounding error."""
    got = np.asarray(got, np.float64).ravel(); ref = np.asarray(ref, np.float64).ravel()
    if dtype == "bf16":
        ulp = np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7
        bad = np.abs(got - ref) > ulp + 1e-30
        assert not bad.any(), f"{what}: {bad.sum()} elements beyond one bf16 ulp, e.g. {got[bad][:4]} vs {ref[bad][:4]}"
        assert rel(got, ref) < 4e-3, f"{what}: rel {rel(got, ref)}"
    else:
        assert rel(got, ref) < 1e-5, f"{what}: rel {rel(got, ref)}"
