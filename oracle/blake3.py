"""BLAKE3 restated in pure Python: the checker of the library's corpus
fingerprint (sj_blake3_*; the reference hashes its corpus with the `blake3`
crate 1.8.7, crates/sejong-train/src/lib.rs:32-56, Cargo.lock:124-127).

TEST INFRASTRUCTURE ONLY: imported by tests/, never by sejong_amd/.

Restated from the published BLAKE3 specification (2020): the 7-round
compression function over a 4 x 4 word state with the message permutation
between rounds, 64-byte blocks in 1024-byte chunks, and the binary tree of
parent nodes whose root output is the hash.  This restatement builds the
tree from the list of all chunk chaining values (split left at the largest
power of two below the chunk count, as the specification defines the tree)
rather than with the incremental stack the library uses, so the two agree
only if both follow the specification.  Pinned in tests/test_oracle.py by
the specification's digests of the empty input and "abc" and by the
reference's recorded fingerprints of its own corpora.
"""
from __future__ import annotations

MASK = 0xFFFFFFFF
IV = (0x6A09E667, 0xBB67AE85, 0x3C6EF372, 0xA54FF53A, 0x510E527F, 0x9B05688C, 0x1F83D9AB, 0x5BE0CD19)
PERM = (2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8)
CHUNK_START, CHUNK_END, PARENT, ROOT = 1, 2, 4, 8
BLOCK, CHUNK = 64, 1024


def _rotr(x, n):
    return ((x >> n) | (x << (32 - n))) & MASK


def _g(s, a, b, c, d, x, y):
    s[a] = (s[a] + s[b] + x) & MASK
    s[d] = _rotr(s[d] ^ s[a], 16)
    s[c] = (s[c] + s[d]) & MASK
    s[b] = _rotr(s[b] ^ s[c], 12)
    s[a] = (s[a] + s[b] + y) & MASK
    s[d] = _rotr(s[d] ^ s[a], 8)
    s[c] = (s[c] + s[d]) & MASK
    s[b] = _rotr(s[b] ^ s[c], 7)


def compress(cv, words, counter, length, flags):
    """16 output words."""
    s = list(cv) + list(IV[:4]) + [counter & MASK, (counter >> 32) & MASK, length, flags]
    m = list(words)
    for r in range(7):
        for i in range(4):
            _g(s, i, 4 + i, 8 + i, 12 + i, m[2 * i], m[2 * i + 1])
        for i in range(4):
            _g(s, i, 4 + (i + 1) % 4, 8 + (i + 2) % 4, 12 + (i + 3) % 4, m[8 + 2 * i], m[9 + 2 * i])
        m = [m[p] for p in PERM]
    return [s[i] ^ s[i + 8] for i in range(8)] + [s[i + 8] ^ cv[i] for i in range(8)]


def _words(block: bytes):
    block = block + bytes(BLOCK - len(block))
    return [int.from_bytes(block[4 * i:4 * i + 4], "little") for i in range(16)]


def _chunk_node(data: bytes, index: int):
    """(cv, words, counter, length, flags) of a chunk's last block, with the
    earlier blocks already compressed into cv."""
    blocks = [data[i:i + BLOCK] for i in range(0, len(data), BLOCK)] or [b""]
    cv = list(IV)
    for j, b in enumerate(blocks[:-1]):
        cv = compress(cv, _words(b), index, BLOCK, CHUNK_START if j == 0 else 0)[:8]
    last = blocks[-1]
    flags = (CHUNK_START if len(blocks) == 1 else 0) | CHUNK_END
    return cv, _words(last), index, len(last), flags


def _parent_node(left, right):
    return list(IV), list(left) + list(right), 0, BLOCK, PARENT


def _cv(node):
    return compress(*node)[:8]


def _subtree(chunks, first):
    """The node of the subtree over `chunks` (their data), the first of
    which has chunk index `first`."""
    if len(chunks) == 1:
        return _chunk_node(chunks[0], first)
    left = 1 << ((len(chunks) - 1).bit_length() - 1)  # largest power of two below the count
    return _parent_node(_cv(_subtree(chunks[:left], first)), _cv(_subtree(chunks[left:], first + left)))


def blake3(data: bytes) -> bytes:
    data = bytes(data)
    chunks = [data[i:i + CHUNK] for i in range(0, len(data), CHUNK)] or [b""]
    cv, words, counter, length, flags = _subtree(chunks, 0)
    out = compress(cv, words, counter, length, flags | ROOT)
    return b"".join(w.to_bytes(4, "little") for w in out[:8])


def corpus_fingerprint(documents) -> str:
    """Corpus::open's hash (lib.rs:32-44): the domain string, then per
    non-empty document its u64 little-endian length and its bytes."""
    parts = [b"Sejong byte corpus v1: EOS + document bytes + EOS"]
    for d in documents:
        d = bytes(d)
        if len(d) == 0:
            continue
        parts += [len(d).to_bytes(8, "little"), d]
    return blake3(b"".join(parts)).hex()
