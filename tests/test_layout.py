"""Host-side layout logic and the C ABI surface, without a GPU: the tile
layout's bijection, the NPU-order permutation the GPU tests use, and that
libggml-zest.so loads and exports every entry point include/*.h declares."""
from __future__ import annotations

import ctypes
import hashlib
import re

import numpy as np
import pytest
from gen import make_data
from helpers import GOLDEN, ROOT, load_pkg
from layout_ref import a_block_index, b_block_index, to_npu_order

GOLD = np.load(GOLDEN / "bfp16_golden.npz")


@pytest.mark.parametrize("M,K,m,k", [(512, 256, 128, 64), (256, 384, 64, 128), (1024, 6144, 128, 64)])
def test_npu_order_permutation_matches_reference(oracle, M, K, m, k):
    x = make_data(M * K, 1 + M + K).reshape(M, K)
    got = to_npu_order(oracle.encode_rows(x), a_block_index(M, K, m, k))
    assert hashlib.sha256(got.tobytes()).digest() == GOLD[f"a_{M}x{K}_m{m}k{k}_sha256"].tobytes()


@pytest.mark.parametrize("N,K,n,k,cols", [(1024, 256, 64, 64, 8), (512, 128, 32, 64, 4)])
def test_npu_b_order_permutation_matches_reference(oracle, N, K, n, k, cols):
    w = make_data(N * K, 7 + N + K).reshape(N, K)
    got = to_npu_order(oracle.encode_rows(w), b_block_index(N, K, n, k, cols))
    assert np.array_equal(got, GOLD[f"b_{N}x{K}_n{n}k{k}c{cols}"])


@pytest.mark.parametrize("rows,k", [(1, 8), (16, 64), (300, 200), (257, 2560)])
def test_tile_layout_round_trip(rows, k):
    z = load_pkg()
    rng = np.random.default_rng(rows * 7 + k)
    blocks = rng.integers(0, 256, size=(rows, k // 8, 9), dtype=np.uint8)
    tiles = z.blocks_to_tiles(blocks, rows, k)
    assert tiles.size == z.bfp16_bytes(rows, k)
    assert np.array_equal(z.tiles_to_blocks(tiles, rows, k), blocks)


def test_tile_layout_offsets():
    # block (r, cb): tile (r/16, cb/8) at (kc * R_pad/16 + rt) * 1152; mantissas
    # at + (r%16)*64 + (cb%8)*8, exponent at + 1024 + (r%16)*8 + cb%8
    z = load_pkg()
    rows, k = 40, 192
    blocks = np.zeros((rows, k // 8, 9), dtype=np.uint8)
    r, cb = 37, 17
    blocks[r, cb] = np.arange(1, 10, dtype=np.uint8)
    tiles = z.blocks_to_tiles(blocks, rows, k)
    rp = z.rows_pad(rows)
    base = ((cb // 8) * (rp // 16) + r // 16) * 1152
    assert tiles[base + 1024 + (r % 16) * 8 + cb % 8] == 1
    assert np.array_equal(tiles[base + (r % 16) * 64 + (cb % 8) * 8: base + (r % 16) * 64 + (cb % 8) * 8 + 8],
                          np.arange(2, 10, dtype=np.uint8))
    assert tiles.sum() == sum(range(1, 10))


def _declared_functions() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(?:ZEST_API|GGML_BACKEND_API)\s+[\w\s\*]+?\b(\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    z = load_pkg()
    lib = z.lib()
    names = _declared_functions()
    assert {"zest_gemm", "zest_pack_act", "zest_convert_weight"} <= names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # the ctypes signatures the package uses cover the zest_* ABI
    assert {n for n in names if n.startswith("zest_")} <= set(z.SIGNATURES)


def test_layout_helpers_agree_with_library():
    z = load_pkg()
    lib = z.lib()
    for rows, k in [(1, 8), (255, 64), (256, 72), (2048, 9728), (4096, 17408)]:
        assert lib.zest_rows_pad(rows) == z.rows_pad(rows)
        assert lib.zest_k_pad(k) == z.k_pad(k)
        assert lib.zest_bfp16_bytes(rows, k) == z.bfp16_bytes(rows, k)
    for t, k in [(0, 2560), (8, 2560), (12, 2560), (8, 9728), (12, 17408)]:
        assert lib.zest_raw_row_bytes(t, k) == z.raw_row_bytes(t, k)


def test_argument_errors_are_reported_without_a_gpu():
    z = load_pkg()
    lib = z.lib()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.zest_pack_act(p, 4, 12, 12, p, None) == -1  # K % 8 != 0
    assert b"multiple of 8" in lib.zest_last_error()
    assert lib.zest_convert_weight(3, p, 4, 64, p, None) != 0  # Q4_1 has no converter
    assert lib.zest_gemm(None, 1, p, 1, 8, p, 1, None, None) == -1
