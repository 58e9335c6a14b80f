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
    assert lib.zest_convert_weight(15, p, 4, 256, p, None) == -3  # Q8_K has no converter
    assert lib.zest_gemm(None, 1, p, 1, 8, p, 1, None, None) == -1


def test_every_entry_point_rejects_bad_arguments_before_the_gpu():
    # Each call below breaks exactly one rule of its entry point's contract
    # (a null or misaligned pointer, a size, a stride, a type or kind), so
    # it must be refused with its code and a message naming the call before
    # anything reaches the GPU: no call here may ever launch (the pointers
    # are host memory).
    z = load_pkg()
    lib = z.lib()
    raw = ctypes.create_string_buffer(1 << 16)
    base = (ctypes.addressof(raw) + 255) & ~255

    def at(off):
        return ctypes.c_void_p(base + off)

    A, W, C, R, X = at(0), at(4096), at(8192), at(12288), at(16384)  # 256-byte aligned
    MIS16, MIS4 = at(4), at(2)
    E_ARG, E_UNSUPPORTED = -1, -3
    f32 = ctypes.c_float
    ptrs = lambda *p: (ctypes.c_void_p * len(p))(*p)  # noqa: E731
    i64s = lambda *v: (ctypes.c_int64 * len(v))(*v)  # noqa: E731
    cases = [
        ("zest_pack_act", (None, 4, 16, 16, A, None), E_ARG),
        ("zest_pack_act", (A, 0, 16, 16, A, None), E_ARG),
        ("zest_pack_act", (A, 4, 12, 12, A, None), E_ARG),          # K % 8
        ("zest_pack_act", (A, 4, 16, 8, A, None), E_ARG),           # ldx < K
        ("zest_pack_act", (MIS16, 4, 16, 16, A, None), E_ARG),
        ("zest_pack_act_x", (A, 4, 16, 16, MIS16, None), E_ARG),
        ("zest_expand_act", (A, 4, 12, A, None), E_ARG),
        ("zest_expand_act", (A, 4, 16, MIS16, None), E_ARG),
        ("zest_convert_weight", (12, None, 4, 256, W, None), E_ARG),
        ("zest_convert_weight", (12, W, 4, 128, W, None), E_ARG),   # Q4_K: K % 256
        ("zest_convert_weight", (12, W, 4, 256, MIS16, None), E_ARG),
        ("zest_convert_weight", (12, MIS4, 4, 256, W, None), E_ARG),  # Q4_K rows 16-byte aligned
        ("zest_convert_weight", (15, W, 4, 256, W, None), E_UNSUPPORTED),  # Q8_K
        ("zest_convert_weight", (0, W, 4, 0, W, None), E_ARG),
        ("zest_convert_weight_gu", (12, W, W, 48, 256, X, None), E_ARG),  # F % 32
        ("zest_convert_weight_gu", (12, W, None, 32, 256, X, None), E_ARG),
        ("zest_convert_weight_gu", (12, W, W, 32, 256, MIS16, None), E_ARG),
        ("zest_gemm", (None, 4, W, 8, 64, C, 8, None, None), E_ARG),
        ("zest_gemm", (A, 4, W, 8, 60, C, 8, None, None), E_ARG),   # K % 8
        ("zest_gemm", (A, 4, W, 8, 64, C, 4, None, None), E_ARG),   # ldc < N
        ("zest_gemm", (A, 0, W, 8, 64, C, 8, None, None), E_ARG),
        ("zest_gemm", (MIS16, 4, W, 8, 64, C, 8, None, None), E_ARG),
        ("zest_gemm", (A, 4, MIS16, 8, 64, C, 8, None, None), E_ARG),
        ("zest_gemm", (A, 4, W, 8, 64, MIS4, 8, None, None), E_ARG),
        ("zest_gemm", (A, 4, W, 8, 64, C, 8, MIS4, None), E_ARG),   # nonfinite
        ("zest_gemm_group", (A, 4, 64, 0, ptrs(W), i64s(8), ptrs(C), i64s(8), None, None), E_ARG),
        ("zest_gemm_group", (A, 4, 64, 5, ptrs(W, W, W, W, W), i64s(8, 8, 8, 8, 8), ptrs(C, C, C, C, C),
                             i64s(8, 8, 8, 8, 8), None, None), E_ARG),
        ("zest_gemm_group", (A, 4, 64, 2, ptrs(W, None), i64s(8, 8), ptrs(C, C), i64s(8, 8), None, None), E_ARG),
        ("zest_gemm_group", (A, 4, 64, 2, ptrs(W, W), i64s(8, 0), ptrs(C, C), i64s(8, 8), None, None), E_ARG),
        ("zest_gemm_group_noalloc", (A, 4, 64, 1, ptrs(W), i64s(8), ptrs(C), i64s(4), None, None), E_ARG),
        ("zest_gemm_group_noalloc", (A, 4, 64, 1, ptrs(MIS16), i64s(8), ptrs(C), i64s(8), None, None), E_ARG),
        ("zest_gemm_residual", (A, 4, W, 8, 64, None, 8, C, 8, None, None), E_ARG),
        ("zest_gemm_residual", (A, 4, W, 8, 64, MIS16, 8, C, 8, None, None), E_ARG),  # residual rows 16-aligned
        ("zest_gemm_residual", (A, 4, W, 8, 64, R, 6, C, 8, None, None), E_ARG),      # ldr % 4
        ("zest_gemm_residual", (A, 4, W, 8, 64, R, 8, C, 4, None, None), E_ARG),      # ldc < N
        ("zest_gemm_residual", (A, 4, MIS16, 8, 64, R, 8, C, 8, None, None), E_ARG),
        ("zest_gemm_glu", (2, A, 4, W, 48, 64, X, None, 0, None, None), E_ARG),       # F % 32
        ("zest_gemm_glu", (2, A, 4, W, 32, 64, None, None, 0, None, None), E_ARG),    # no output
        ("zest_gemm_glu", (2, A, 4, W, 32, 64, None, C, 16, None, None), E_ARG),      # ldh < F
        ("zest_gemm_glu", (2, A, 4, W, 32, 64, MIS16, None, 0, None, None), E_ARG),
        ("zest_gemm_glu", (2, A, 4, W, 32, 64, X, MIS4, 32, None, None), E_ARG),
        ("zest_gemm_glu", (7, A, 4, W, 32, 64, X, None, 0, None, None), E_UNSUPPORTED),  # kind
        ("zest_rms_norm", (None, 4, 16, f32(1e-6), None, C, None, None), E_ARG),
        ("zest_rms_norm", (A, 4, 16, f32(1e-6), None, None, None, None), E_ARG),      # no output
        ("zest_rms_norm", (A, 0, 16, f32(1e-6), None, C, None, None), E_ARG),
        ("zest_rms_norm", (A, 4, 12, f32(1e-6), None, None, X, None), E_ARG),         # packing: d % 8
        ("zest_rms_norm", (A, 4, 16, f32(1e-6), None, None, MIS16, None), E_ARG),
        ("zest_glu", (2, A, 16, W, 16, 4, 16, None, None, None), E_ARG),              # no output
        ("zest_glu", (2, A, 8, W, 16, 4, 16, C, None, None), E_ARG),                  # sg < f
        ("zest_glu", (2, A, 16, W, 16, 4, 12, None, X, None), E_ARG),                 # packing: f % 8
        ("zest_glu", (2, A, 16, W, 16, 4, 16, None, MIS16, None), E_ARG),
        ("zest_glu", (3 + 7, A, 16, W, 16, 4, 16, C, None, None), E_UNSUPPORTED),     # kind
        ("zest_add", (A, None, 4, 16, 0, C, None), E_ARG),
        ("zest_add", (A, W, 4, 0, 0, C, None), E_ARG),
        ("zest_mul_row", (A, W, 0, 16, C, None), E_ARG),
        ("zest_scale", (A, 0, f32(1.0), f32(0.0), C, None), E_ARG),
        ("zest_scale", (A, 16, f32(1.0), f32(0.0), None, None), E_ARG),
        ("zest_rope", (A, 4, 2, 64, None, None, 64, 0, f32(1e4), f32(1), f32(0), f32(1), f32(0), f32(0), C, None),
         E_ARG),                                                                      # no positions
        ("zest_rope", (A, 4, 2, 64, R, None, 63, 0, f32(1e4), f32(1), f32(0), f32(1), f32(0), f32(0), C, None),
         E_ARG),                                                                      # odd n_dims
        ("zest_rope", (A, 4, 2, 64, R, None, 128, 0, f32(1e4), f32(1), f32(0), f32(1), f32(0), f32(0), C, None),
         E_ARG),                                                                      # n_dims > d
        ("zest_rope", (A, 4, 2, 64, R, None, 64, 1, f32(1e4), f32(1), f32(0), f32(1), f32(0), f32(0), C, None),
         E_ARG),                                                                      # mode
        ("zest_check_finite", (C, 4, 16, 8, R, None), E_ARG),                         # ld < cols
        ("zest_check_finite", (C, 4, 16, 16, MIS4, None), E_ARG),
    ]
    declared = {n for n in _declared_functions() if n.startswith("zest_")}
    covered = {name for name, _, _ in cases}
    # every entry point that takes device memory has cases here
    assert declared - covered <= {"zest_init", "zest_self_test", "zest_last_error", "zest_rows_pad", "zest_k_pad",
                                  "zest_bfp16_bytes", "zest_act_bytes", "zest_raw_row_bytes", "zest_release_stream"}
    for name, args, want in cases:
        got = getattr(lib, name)(*args)
        msg = lib.zest_last_error().decode()
        assert got == want, f"{name}{args}: returned {got}, wanted {want} ({msg})"
        short = name.replace("zest_gemm_group", "zest_gemm")
        assert msg.startswith(short) or msg.startswith(name), f"{name}: message {msg!r}"
