"""Device-memory helpers for the GPU parity tests.

Device buffers come from the library's own sj_alloc / sj_upload /
sj_download (torch's wheel carries a second HIP runtime; two runtimes in one
process do not share devices or pointers, so torch is not loaded here).
Every computation under test runs in libsejong_hip.so."""
import ctypes

import numpy as np

from oracle import oracle as O


def _api():
    from sejong_amd import _native as N
    N.load()
    return N.api


# Every buffer made by a test stays alive until the autouse fixture in
# conftest releases it after the test has synchronised: a kernel must never
# read memory whose Python owner was already collected.
LIVE = []


class Dev:
    """A device buffer with a dtype tag ('f32', 'bf16', 'i32', 'f64', 'u8')."""

    ITEM = {"f32": 4, "bf16": 2, "i32": 4, "f64": 8, "u8": 1}

    def __init__(self, n: int, dtype: str = "f32"):
        self.n, self.dtype = int(n), dtype
        self.nbytes = max(self.n * self.ITEM[dtype], 1)
        p = ctypes.c_void_p()
        _api().sj_alloc(self.nbytes, ctypes.byref(p))
        self.ptr = p.value
        LIVE.append(self)

    def __del__(self):
        try:
            if self.ptr:
                _api().sj_free(ctypes.c_void_p(self.ptr))
                self.ptr = None
        except Exception:
            pass

    @property
    def p(self):
        return ctypes.c_void_p(self.ptr)

    def at(self, elements: int):
        """Pointer `elements` into the buffer."""
        return ctypes.c_void_p(self.ptr + elements * self.ITEM[self.dtype])

    def upload(self, values):
        a = np.ascontiguousarray(values)
        if self.dtype == "bf16":
            raw = (a.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        elif self.dtype == "f32":
            raw = a.astype(np.float32)
        elif self.dtype == "i32":
            raw = a.astype(np.int32)
        elif self.dtype == "f64":
            raw = a.astype(np.float64)
        else:
            raw = a.astype(np.uint8)
        raw = np.ascontiguousarray(raw).ravel()
        assert raw.nbytes <= self.nbytes
        _api().sj_upload(self.p, ctypes.c_void_p(raw.ctypes.data), raw.nbytes)
        return self

    def host(self) -> np.ndarray:
        if self.dtype == "bf16":
            raw = np.empty(self.n, np.uint16)
        else:
            raw = np.empty(self.n, {"f32": np.float32, "i32": np.int32, "f64": np.float64, "u8": np.uint8}[self.dtype])
        _api().sj_download(ctypes.c_void_p(raw.ctypes.data), self.p, raw.nbytes)
        if self.dtype == "bf16":
            return (raw.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        return raw.astype(np.float64) if self.dtype in ("f32", "f64") else raw


def dev(x, dtype="f32"):
    """Upload values as a new device buffer.  bf16 inputs must already be
    bf16-representable (use O.round_to); they are truncated to bf16 bits."""
    a = np.asarray(x)
    return Dev(a.size, dtype).upload(a)


def empty(n, dtype="f32"):
    return Dev(n, dtype)


def zeros(n, dtype="f32"):
    return Dev(n, dtype).upload(np.zeros(n))


def sync():
    _api().sj_synchronize(None)


def rnd(shape, dtype, rng, std=1.0):
    """Random values already rounded to the storage dtype."""
    return O.round_to(rng.normal(0, std, shape), dtype)


def rel(a, b):
    a = np.asarray(a, np.float64).ravel(); b = np.asarray(b, np.float64).ravel()
    n = np.linalg.norm(b)
    return np.linalg.norm(a - b) / (n if n > 0 else 1.0)


def release_all():
    _api().sj_synchronize(None)
    LIVE.clear()


def assert_stored_close(got, ref, dtype, what="", ulps=1.0, terms=None):
    """`got` was stored in `dtype`; `ref` is the FP64 value before that
    store.  Each element must lie within `ulps` storage ulps of ref (device
    and oracle may round a near-tie to different neighbours) plus the fp32
    accumulation error 2^-16 * terms, where `terms` is the sum of |products|
    that formed the element (cancellation leaves a result far below its
    terms); the tensor as a whole must be within the storage rounding error."""
    got = np.asarray(got, np.float64).ravel(); ref = np.asarray(ref, np.float64).ravel()
    acc = 0.0 if terms is None else 2.0 ** -16 * np.asarray(terms, np.float64).ravel()
    if dtype == "bf16":
        tol = np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7 * ulps + acc
        bad = np.abs(got - ref) > tol + 1e-30
        assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} elements beyond {ulps} bf16 ulp, e.g. {got[bad][:4]} vs {ref[bad][:4]}"
        assert rel(got, ref) < 4e-3, f"{what}: rel {rel(got, ref)}"
    else:
        assert rel(got, ref) < 1e-5, f"{what}: rel {rel(got, ref)}"
