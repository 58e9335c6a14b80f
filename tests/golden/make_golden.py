"""Writes tests/golden/bfp16_golden.npz from the reference's own bfp16 packer.

The packer is compiled from the reference's source (src/npu/bfp16_pack.cpp)
by oracle/Makefile into oracle/_ref/, once with AVX2 (the production path)
and once scalar. Inputs come from gen.py (deterministic), so a fixture
stores only the reference's output bytes (or, for the large shapes of
tests/test-bfp16-pack.cpp:101 and :134-135, their sha256).

    python tests/golden/make_golden.py      # needs oracle/_ref built
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(HERE.parent))

from gen import edge_blocks, make_data  # noqa: E402
from helpers import RefPacker  # noqa: E402

# tests/test-bfp16-pack.cpp:101 (activations, seed 1+M+K) and :134-135
# (weights, seed 7+N+K); the largest ones are kept as hashes.
A_SHAPES = [(512, 256, 128, 64), (256, 384, 64, 128), (1024, 6144, 128, 64)]
B_SHAPES = [(1024, 256, 64, 64, 8), (4096, 2048, 64, 64, 8), (2048, 6144, 64, 128, 8), (512, 128, 32, 64, 4)]
FULL_BYTES_LIMIT = 300_000


def main() -> None:
    avx2, scalar = RefPacker("avx2"), RefPacker("scalar")
    out: dict[str, np.ndarray] = {}

    blocks = np.concatenate([make_data(1024 * 8, 11).reshape(-1, 8), edge_blocks()])
    enc = avx2.encode_blocks(blocks)
    enc_s = scalar.encode_blocks(blocks)
    assert (enc == enc_s).all(), "AVX2 and scalar reference encoders disagree on finite inputs"
    out["blocks_x"] = blocks
    out["blocks_enc"] = enc

    for M, K, m, k in A_SHAPES:
        x = make_data(M * K, 1 + M + K).reshape(M, K)
        got = avx2.pack_a(x, m, k)
        assert (got == scalar.pack_a(x, m, k)).all()
        key = f"a_{M}x{K}_m{m}k{k}"
        if got.size <= FULL_BYTES_LIMIT:
            out[key] = got
        out[key + "_sha256"] = np.frombuffer(hashlib.sha256(got.tobytes()).digest(), dtype=np.uint8)

    for N, K, n, k, cols in B_SHAPES:
        w = make_data(N * K, 7 + N + K).reshape(N, K)
        got = avx2.pack_b(w, n, k, cols)
        assert (got == scalar.pack_b(w, n, k, cols)).all()
        key = f"b_{N}x{K}_n{n}k{k}c{cols}"
        if got.size <= FULL_BYTES_LIMIT:
            out[key] = got
        out[key + "_sha256"] = np.frombuffer(hashlib.sha256(got.tobytes()).digest(), dtype=np.uint8)

    np.savez_compressed(HERE / "bfp16_golden.npz", **out)
    total = sum(v.nbytes for v in out.values())
    print(f"wrote {HERE / 'bfp16_golden.npz'}: {len(out)} arrays, {total} bytes before compression")


if __name__ == "__main__":
    main()
