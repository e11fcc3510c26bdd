"""Byte corpora for training and evaluation batches (crates/sejong-train/
src/lib.rs:17-102, `Corpus`).

A corpus is the sorted list of non-empty text files under a path, read as
one token stream EOS + document bytes + EOS + document bytes + ... + EOS:
document i occupies the positions (ends[i-1], ends[i]) after its leading EOS
at ends[i-1], and the final position tokens - 1 is the closing EOS.
`batch` draws, per sequence, start = rng.index(tokens - sequence) and takes
inputs start .. start+sequence-1 and targets one position later.  Files are
memory-mapped; token lookup is vectorised over the batch.  `fingerprint` is
the corpus's BLAKE3 hash as Corpus::open forms it (lib.rs:32-56), hashed by
the library's host code; checkpoints record it as data_fingerprint and a
resume refuses a different corpus (lib.rs:338-341, 478-483).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import _native as N
from .model import EOS
from .rng import Rng

FINGERPRINT_DOMAIN = b"Sejong byte corpus v1: EOS + document bytes + EOS"


def fingerprint(documents) -> str:
    """Corpus::open's hash (lib.rs:32-44): BLAKE3 of the domain string, then
    per non-empty document its u64 little-endian length and its bytes."""
    N.load()
    state = ctypes.create_string_buffer(N.api.sj_blake3_state_bytes() + 8)
    st = ctypes.c_void_p((ctypes.addressof(state) + 7) // 8 * 8)
    N.api.sj_blake3_init(st)
    N.api.sj_blake3_update(st, FINGERPRINT_DOMAIN, len(FINGERPRINT_DOMAIN))
    for d in documents:
        a = np.ascontiguousarray(d, dtype=np.uint8)
        if a.size == 0:
            continue
        n = np.array([a.size], dtype="<u8")
        N.api.sj_blake3_update(st, ctypes.c_void_p(n.ctypes.data), 8)
        N.api.sj_blake3_update(st, ctypes.c_void_p(a.ctypes.data), a.size)
    out = (ctypes.c_uint8 * 32)()
    N.api.sj_blake3_finalize(st, out)
    return bytes(out).hex()


def _collect_text(path: str, files: list):
    """collect_text (lib.rs:89-109): a file path is taken as it is; a
    directory contributes its *.txt files, recursively; anything else is an
    error."""
    if os.path.isfile(path):
        files.append(path)
    elif os.path.isdir(path):
        for entry in os.listdir(path):
            p = os.path.join(path, entry)
            if os.path.isdir(p):
                _collect_text(p, files)
            elif os.path.splitext(entry)[1] == ".txt":
                files.append(p)
    else:
        raise ValueError(f"corpus path does not exist: {path}")


def _path_key(p: str):
    # PathBuf ordering compares path components, not the joined string
    return tuple(os.fsencode(part) for part in p.split(os.sep) if part not in ("", "."))


class Corpus:
    """Corpus::open / token / batch (lib.rs:23-88)."""

    def __init__(self, documents: list):
        self.documents = [np.asarray(d, dtype=np.uint8) for d in documents if len(d) > 0]
        lengths = np.array([d.size + 1 for d in self.documents], dtype=np.int64)
        self.ends = np.cumsum(lengths)
        total = int(self.ends[-1]) if self.ends.size else 0
        if total <= 1:
            raise ValueError("corpus contains no text")
        self.tokens = total + 1
        self._flat = np.concatenate(self.documents) if self.documents else np.zeros(0, np.uint8)
        # start of each document's bytes in the concatenation of all documents
        self._flat_start = np.concatenate([[0], np.cumsum([d.size for d in self.documents])])[:-1]
        self.fingerprint = fingerprint(self.documents)

    @classmethod
    def open(cls, path: str) -> "Corpus":
        files: list = []
        _collect_text(os.fspath(path), files)
        files.sort(key=_path_key)
        if not files:
            raise ValueError("corpus requires at least one text file")
        docs = []
        for f in files:
            if os.path.getsize(f) == 0:
                continue
            docs.append(np.memmap(f, dtype=np.uint8, mode="r"))
        return cls(docs)

    def token_array(self, index) -> np.ndarray:
        """token(index) for an array of stream positions (lib.rs:59-71)."""
        index = np.asarray(index, dtype=np.int64)
        if index.size and (index.min() < 0 or index.max() >= self.tokens):
            raise IndexError("corpus position out of range")
        doc = np.searchsorted(self.ends, index, side="right")   # partition_point(end <= index)
        last = index == self.tokens - 1
        docc = np.minimum(doc, len(self.documents) - 1)
        start = np.where(doc == 0, 0, self.ends[np.maximum(doc - 1, 0)])
        local = index - start
        at = np.clip(self._flat_start[docc] + local - 1, 0, max(self._flat.size - 1, 0))
        byte = self._flat[at].astype(np.int32)
        return np.where(last | (local == 0), np.int32(EOS), byte).astype(np.int32)

    def token(self, index: int) -> int:
        return int(self.token_array(np.array([index]))[0])

    def batch(self, rng: Rng, batch: int, sequence: int) -> tuple[np.ndarray, np.ndarray]:
        """Corpus::batch (lib.rs:72-88): inputs and targets [batch * sequence]."""
        if sequence <= 0 or self.tokens - sequence <= 0:
            raise ValueError("corpus is shorter than one sequence")
        starts = np.array([rng.index(self.tokens - sequence) for _ in range(batch)], dtype=np.int64)
        pos = starts[:, None] + np.arange(sequence, dtype=np.int64)[None, :]
        return self.token_array(pos).reshape(-1), self.token_array(pos + 1).reshape(-1)
