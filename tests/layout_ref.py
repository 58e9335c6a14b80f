"""The reference's NPU operand order as a vectorised numpy permutation, used by
the tests to carry row-major blocks (what our tile layout maps to through
tiles_to_blocks) into the byte order of the reference's packer output.

Offsets restate bfp16_a_offset / bfp16_b_offset (src/npu/bfp16_pack.cpp:
286-302); test_layout.py checks this module against the oracle and the
reference packer's golden bytes before any GPU test relies on it."""
from __future__ import annotations

import numpy as np


def _in_tile(rr, cb, k):
    tkb = k // 8
    return ((rr // 16) * tkb + cb % tkb) * 16 + rr % 16


def a_block_index(M: int, K: int, m: int, k: int) -> np.ndarray:
    r = np.arange(M)[:, None]
    cb = np.arange(K // 8)[None, :]
    nk = K // k
    tile = (r // m) * nk + cb // (k // 8)
    return tile * m * (k // 8) + _in_tile(r % m, cb, k)


def b_block_index(N: int, K: int, n: int, k: int, cols: int) -> np.ndarray:
    r = np.arange(N)[:, None]
    cb = np.arange(K // 8)[None, :]
    per_col, nk, g = N // n // cols, K // k, r // n
    tile = ((g % cols) * per_col + g // cols) * nk + cb // (k // 8)
    return tile * n * (k // 8) + _in_tile(r % n, cb, k)


def to_npu_order(blocks: np.ndarray, index: np.ndarray) -> np.ndarray:
    """blocks [R][K/8][9] row-major -> the NPU byte stream."""
    out = np.empty((index.size, 9), dtype=np.uint8)
    out[index.reshape(-1)] = blocks.reshape(-1, 9)
    return out.reshape(-1)
