"""SplitMix64 `Rng` of crates/sejong-core/src/lib.rs:591-623, vectorised.

next_u64 advances the state by the golden-gamma increment and mixes it, so
a block of n draws is a pure function of (state, n) and is computed with
numpy uint64 arithmetic.  index() keeps the reference's rejection rule.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_MASK = (1 << 64) - 1


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


class Rng:
    def __init__(self, seed: int):
        self.state = int(seed) & _MASK

    def next_block(self, n: int) -> np.ndarray:
        """n consecutive next_u64() draws (lib.rs:600-606)."""
        steps = np.arange(1, n + 1, dtype=np.uint64)
        with np.errstate(over="ignore"):
            states = np.uint64(self.state) + steps * _GAMMA
        self.state = (self.state + n * 0x9E3779B97F4A7C15) & _MASK
        return _mix(states)

    def next_u64(self) -> int:
        return int(self.next_block(1)[0])

    def index(self, size: int) -> int:
        """Rejection-sampled index in [0, size) (lib.rs:610-619)."""
        n = int(size)
        threshold = ((1 << 64) - n) % n
        while True:
            x = self.next_u64()
            if x >= threshold:
                return x % n

    def indices(self, size: int, count: int) -> np.ndarray:
        """count successive index(size) draws."""
        n = int(size)
        threshold = ((1 << 64) - n) % n
        if threshold == 0:  # powers of two (e.g. bytes): no rejection possible
            return (self.next_block(count) % np.uint64(n)).astype(np.int64)
        return np.array([self.index(n) for _ in range(count)], dtype=np.int64)

    def uniform(self, count: int) -> np.ndarray:
        """Rng::uniform as float64 ((x >> 40) + 0.5) / 2^24 (lib.rs:607-609)."""
        return ((self.next_block(count) >> np.uint64(40)).astype(np.float64) + 0.5) / 16777216.0

    def normal(self, count: int, std: float = 1.0) -> np.ndarray:
        """Box-Muller in double from pairs of uniform draws."""
        u = self.uniform(2 * count)
        u1, u2 = u[0::2], u[1::2]
        return std * np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
