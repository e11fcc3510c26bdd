"""NativeValue host logic (no GPU): request packing, the value parameters'
layout and the request sampler's RNG stream."""
import numpy as np

from sejong_amd.model import ModelConfig, layout, value_layout
from sejong_amd.rng import Rng
from sejong_amd.value import BOS, PAD, SAMPLE_SEED, SEP, initial_params, pack


def test_pack_rows_and_sep_positions():
    ids, sel = pack([b"ab", b"xyz", b""], [1, 0, 2], 6)
    np.testing.assert_array_equal(ids.reshape(3, 6), [[BOS, 120, 121, 122, SEP, PAD], [BOS, 97, 98, SEP, PAD, PAD],
                                                      [BOS, SEP, PAD, PAD, PAD, PAD]])
    np.testing.assert_array_equal(sel, [4, 9, 13])


def test_value_layout_and_init():
    mc = ModelConfig(width=64, layers=2, heads=2, kv_heads=1, ffn_width=96, context=32)
    names = [n for n, _, _ in value_layout(mc, 7)]
    assert names[-3:] == ["native_embedding", "native_value", "native_bias"]
    assert "embedding" not in names and "output" not in names
    assert names[:-3] == [n for n, _, _ in layout(mc)][1:-1]
    p = initial_params(mc, 7)
    assert p.size == sum(int(np.prod(s)) for _, s, _ in value_layout(mc, 7))
    assert np.all(p[-7:] == 0)                       # bias starts at zero
    emb = p[-(7 + 64 * 7 + 259 * 64):-(7 + 64 * 7)]
    assert abs(emb.std() * 8 - 1) < 0.05             # normal / sqrt(d)


def test_sampler_stream():
    from sejong_amd.model import TrainConfig
    r = Rng(42 ^ SAMPLE_SEED)
    expect = [r.index(12) for _ in range(5)]
    r2 = Rng(42 ^ SAMPLE_SEED)
    assert [r2.index(12) for _ in range(5)] == expect
