"""Deterministic input generators shared by the golden-vector script and the
tests: a splitmix64 counter generator with Box-Muller normals, so the same
seed gives the same floats on every machine and numpy version."""
from __future__ import annotations

import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


class Rng:
    def __init__(self, seed: int):
        with np.errstate(over="ignore"):
            self.ctr = np.uint64(seed) * _GOLD

    def u64(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            idx = (np.arange(1, n + 1, dtype=np.uint64) * _GOLD) + self.ctr
            self.ctr = self.ctr + np.uint64(n) * _GOLD
            return _mix(idx)

    def uniform(self, n: int) -> np.ndarray:
        """(0, 1] doubles."""
        return ((self.u64(n) >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)

    def normal(self, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        u1, u2 = self.uniform(n), self.uniform(n)
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        return (mean + std * z).astype(np.float32)

    def ints(self, n: int, lo: int, hi: int) -> np.ndarray:
        """Integers in [lo, hi]."""
        return (lo + (self.u64(n) % np.uint64(hi - lo + 1)).astype(np.int64)).astype(np.int64)


def make_data(n: int, seed: int) -> np.ndarray:
    """The mixture tests/test-bfp16-pack.cpp:77-91 builds, with this module's
    generator: exact zeros, 127.75*2^e (rounds past 127 when it is a block's
    maximum), ties (0.5 + j)*2^e, and normals scaled by 2^e, e in [-24, 12]."""
    rng = Rng(seed)
    kind = rng.ints(n, 0, 9)
    e = rng.ints(n, -24, 12)
    tie = 0.5 + rng.ints(n, 0, 63).astype(np.float32)
    nd = rng.normal(n)
    x = np.where(kind == 0, 0.0, np.where(kind == 1, 127.75, np.where(kind == 2, tie, nd))).astype(np.float32)
    return np.ldexp(x, e.astype(np.int32)).astype(np.float32)


def wide_blocks(rows: int, k: int, seed: int, std: float = 1.0) -> np.ndarray:
    """N(0, std) values [rows][k] with each 8-value block along k scaled by
    2^U(-12, 12): products of two such operands span about 2^48, so fp32
    partial sums of them are rarely exact and summing K in another order
    (another split of K among workgroups) changes bits. Operands for tests
    that claim two launches sum in the same order."""
    rng = Rng(seed)
    x = rng.normal(rows * k, 0.0, std).reshape(rows, k // 8, 8)
    e = rng.ints(rows * (k // 8), -12, 12).reshape(rows, k // 8, 1).astype(np.int32)
    return np.ldexp(x, e).reshape(rows, k).astype(np.float32)


def edge_blocks() -> np.ndarray:
    """Blocks that take the encoder's special paths: all zeros and negative
    zeros, subnormal-only blocks (exponent byte 0), tiny normals (bytes 1..6,
    where 2^(133-e) is not a normal float), the saturation KAT block of
    tests/test-bfp16-pack.cpp:169-170, ties at every position, and blocks
    near FLT_MAX. Finite values only."""
    b = []
    b.append([0.0, -0.0, 0.0, 0.0, -0.0, 0.0, 0.0, 0.0])
    b.append([-0.0] * 8)
    sub = np.float32(1.0e-40)
    b.append([sub, -sub, sub * 3, 0.0, -sub * 7, sub * 100, 1.4e-45, -1.4e-45])
    for e in range(1, 8):
        v = np.ldexp(np.float32(1.0), e - 127)
        b.append([v, -v * 1.5, v * 1.9, v * 0.25, -v * 0.126, v * 1.0001, 0.0, -v])
    sat = np.ldexp(np.array([127.75, 1.0, -3.5, 0.0, 64.0, -127.5, 0.25, 100.5], dtype=np.float32), -6)
    b.append(list(sat))
    for p in range(8):
        row = [0.5] * 8
        row[p] = 64.0  # max 64 -> exponent 133, step 1/... ties at .5
        b.append([v * 1.0 for v in row])
    big = np.float32(3.0e38)
    b.append([big, -big, big / 3, 1.0, -1.0, 0.0, big / 1e10, -big / 2])
    b.append([-127.75 * 2.0 ** -6] + [1.0 * 2.0 ** -6] * 7)
    return np.array(b, dtype=np.float32)
