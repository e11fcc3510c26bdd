"""Corpus (crates/sejong-train/src/lib.rs:17-102) on the CPU: file
collection, the EOS-delimited token stream and Corpus::batch, against a
brute-force restatement that builds the whole stream as a list (no
partition_point), with the draws from the oracle's SplitMix64."""
import os

import numpy as np
import pytest

from oracle import blake3 as B3
from oracle import oracle as O
from sejong_amd.corpus import Corpus, fingerprint
from sejong_amd.model import EOS
from sejong_amd.rng import Rng

TRAIN = "/root/reference/docs/measurements/2026-11-01/train.txt"
VALIDATION = "/root/reference/docs/measurements/2026-11-01/validation.txt"


def brute_stream(docs):
    out = []
    for d in docs:
        if len(d) == 0:
            continue
        out.append(EOS)
        out.extend(int(b) for b in d)
    out.append(EOS)
    return out


def brute_batch(stream, seed, batch, sequence):
    rng = O.Rng(seed)
    ids, tg = [], []
    for _ in range(batch):
        start = rng.index(len(stream) - sequence)
        ids += stream[start:start + sequence]
        tg += stream[start + 1:start + sequence + 1]
    return np.array(ids, np.int32), np.array(tg, np.int32)


def test_stream_layout_and_file_collection(tmp_path):
    rng = np.random.default_rng(3)
    (tmp_path / "a").mkdir()
    (tmp_path / "a" / "deep").mkdir()
    files = {
        "a/b.txt": rng.integers(0, 256, 37, dtype=np.uint8),
        "a.txt": rng.integers(0, 256, 5, dtype=np.uint8),
        "a/deep/c.txt": rng.integers(0, 256, 1, dtype=np.uint8),
        "empty.txt": np.zeros(0, np.uint8),               # skipped
        "notes.md": rng.integers(0, 256, 9, dtype=np.uint8),  # not a .txt file
        "z.txt": rng.integers(0, 256, 64, dtype=np.uint8),
    }
    for name, data in files.items():
        (tmp_path / name).write_bytes(data.tobytes())
    c = Corpus.open(tmp_path)
    # PathBuf order compares components: a/b.txt and a/deep/c.txt come before a.txt
    order = ["a/b.txt", "a/deep/c.txt", "a.txt", "z.txt"]
    stream = brute_stream([files[n] for n in order])
    assert c.tokens == len(stream) == sum(files[n].size + 1 for n in order) + 1
    np.testing.assert_array_equal(c.token_array(np.arange(c.tokens)), stream)
    assert c.token(0) == EOS and c.token(c.tokens - 1) == EOS
    for seed, b, t in [(123, 4, 16), (7, 3, 100), (0, 1, len(stream) - 1)]:
        ids, tg = c.batch(Rng(seed), b, t)
        rid, rtg = brute_batch(stream, seed, b, t)
        np.testing.assert_array_equal(ids, rid)
        np.testing.assert_array_equal(tg, rtg)
    # a single file path is taken whatever its extension
    one = Corpus.open(tmp_path / "notes.md")
    assert one.tokens == files["notes.md"].size + 2


def test_errors(tmp_path):
    with pytest.raises(ValueError, match="at least one text file"):
        Corpus.open(tmp_path)
    # collect_text (lib.rs:103-107): a path that is neither file nor directory
    with pytest.raises(ValueError, match="corpus path does not exist: .*missing"):
        Corpus.open(tmp_path / "missing")
    (tmp_path / "e.txt").write_bytes(b"")
    with pytest.raises(ValueError, match="no text"):
        Corpus.open(tmp_path)
    (tmp_path / "f.txt").write_bytes(b"abc")
    c = Corpus.open(tmp_path)
    assert c.tokens == 5
    with pytest.raises(ValueError, match="shorter than one sequence"):
        c.batch(Rng(1), 1, 5)


@pytest.mark.skipif(not os.path.exists(TRAIN), reason="the reference's measurement corpus is not present")
def test_reference_measurement_corpus_seed_123():
    """The corpus of the reference's RX 6600 measurement (16,939 bytes):
    training batches at seed 123 (the data seed of that run) for the bench
    shape (8 x 512) and the cached measurement's single 512-byte sequence."""
    raw = np.fromfile(TRAIN, dtype=np.uint8)
    assert raw.size == 16939
    c = Corpus.open(TRAIN)
    stream = brute_stream([raw])
    assert c.tokens == 16941
    for b, t in [(8, 512), (1, 512), (2, 1024)]:
        ids, tg = c.batch(Rng(123), b, t)
        rid, rtg = brute_batch(stream, 123, b, t)
        np.testing.assert_array_equal(ids, rid)
        np.testing.assert_array_equal(tg, rtg)
    v = Corpus.open(VALIDATION)
    assert v.tokens == 7633 + 2


# the reference's recorded fingerprints of its measurement corpora
# (docs/measurements/2026-11-01/rx6600-learning-window.json:2111,2119)
TRAIN_FINGERPRINT = "b96cc76f31fa0a61e840635e05d1ceea137d68329cbe2d20504b8f34d371943f"
VALIDATION_FINGERPRINT = "9a1409d8fd61e18c2ca1fef712488fbe776e90f3c10fd9a9b88d9eb11503d16e"


@pytest.mark.skipif(not os.path.exists(TRAIN), reason="the reference's measurement corpus is not present")
def test_fingerprint_matches_reference_record():
    """Corpus::open's BLAKE3 fingerprint (lib.rs:32-56) of the reference's
    own training and validation corpora equals the fingerprints its
    measurement recorded (17 and 8 BLAKE3 chunks: parent nodes over
    uneven trees)."""
    assert Corpus.open(TRAIN).fingerprint == TRAIN_FINGERPRINT
    assert Corpus.open(VALIDATION).fingerprint == VALIDATION_FINGERPRINT


def test_library_blake3_against_oracle():
    """The library's incremental BLAKE3 (sj_blake3_*) against the oracle's
    whole-tree restatement at the block and chunk boundaries (1 .. 3 blocks,
    1 .. 2 chunks, tree shapes of 3 .. 100 chunks), fed in one piece and in
    uneven pieces; and the corpus hash over several documents with empty
    ones skipped."""
    import ctypes
    from sejong_amd import _native as N
    N.load()
    rng = np.random.default_rng(11)

    def lib_hash(data, pieces):
        st = ctypes.create_string_buffer(N.api.sj_blake3_state_bytes() + 8)
        p = ctypes.c_void_p((ctypes.addressof(st) + 7) // 8 * 8)
        N.api.sj_blake3_init(p)
        a = np.frombuffer(data, np.uint8) if data else np.zeros(0, np.uint8)
        cuts = sorted(set(int(x) for x in pieces if 0 < x < len(data)))
        for lo, hi in zip([0] + cuts, cuts + [len(data)]):
            N.api.sj_blake3_update(p, ctypes.c_void_p(a.ctypes.data + lo), hi - lo)
        out = (ctypes.c_uint8 * 32)()
        N.api.sj_blake3_finalize(p, out)
        return bytes(out)

    for n in [0, 1, 63, 64, 65, 127, 128, 1023, 1024, 1025, 2048, 2049, 3072, 3073, 4096, 4097, 8193, 31744,
              102400]:
        data = bytes(np.arange(n) % 251 % 256)  # the BLAKE3 test-vector input pattern
        want = B3.blake3(data)
        assert lib_hash(data, []) == want, n
        assert lib_hash(data, rng.integers(0, max(n, 1), 5)) == want, n
        assert lib_hash(data, [64, 1024, 1025]) == want, n
    docs = [rng.integers(0, 256, k, dtype=np.uint8) for k in (5000, 0, 1, 1024, 77)]
    assert fingerprint(docs) == B3.corpus_fingerprint([d.tobytes() for d in docs])
