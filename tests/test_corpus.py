"""Corpus (crates/sejong-train/src/lib.rs:17-102) on the CPU: file
collection, the EOS-delimited token stream and Corpus::batch, against a
brute-force restatement that builds the whole stream as a list (no
partition_point), with the draws from the oracle's SplitMix64."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from sejong_amd.corpus import Corpus
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
