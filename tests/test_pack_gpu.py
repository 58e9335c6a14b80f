"""The HIP activation packer and weight converters against the reference's
golden bytes and the CPU oracle: bit-exact (tests/test-bfp16-pack.cpp's bar),
through the tile layout's bijection to row-major blocks."""
from __future__ import annotations

import hashlib

import numpy as np
import pytest
from gen import Rng, edge_blocks, make_data
from helpers import GOLDEN, load_quant
from layout_ref import a_block_index, b_block_index, to_npu_order

pytestmark = pytest.mark.gpu
GOLD = np.load(GOLDEN / "bfp16_golden.npz")


def gpu_pack(z, x: np.ndarray, ldx: int | None = None) -> np.ndarray:
    import torch
    m, k = x.shape
    if ldx is None:
        xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    else:
        full = torch.zeros((m, ldx), dtype=torch.float32)
        full[:, :k] = torch.from_numpy(x)
        xt = full.cuda()[:, :k]
    out = z.pack_act(xt)
    torch.cuda.synchronize()
    return z.tiles_to_blocks(out.cpu().numpy(), m, k)


@pytest.mark.parametrize("M,K,m,k", [(512, 256, 128, 64), (256, 384, 64, 128), (1024, 6144, 128, 64)])
def test_pack_act_matches_reference_golden(zest_gpu, M, K, m, k):
    x = make_data(M * K, 1 + M + K).reshape(M, K)
    got = to_npu_order(gpu_pack(zest_gpu, x), a_block_index(M, K, m, k))
    key = f"a_{M}x{K}_m{m}k{k}"
    if key in GOLD:
        assert np.array_equal(got, GOLD[key])
    assert hashlib.sha256(got.tobytes()).digest() == GOLD[key + "_sha256"].tobytes()


def test_pack_act_golden_blocks_and_edge_cases(zest_gpu):
    x = GOLD["blocks_x"]  # make_data blocks + zero / subnormal / tiny / saturating / near-FLT_MAX blocks
    n = x.shape[0] // 8 * 8
    got = gpu_pack(zest_gpu, x[:n].reshape(-1, 64))
    assert np.array_equal(got.reshape(-1, 9), GOLD["blocks_enc"][:n])
    e = edge_blocks()
    got = gpu_pack(zest_gpu, e.reshape(1, -1))
    assert np.array_equal(got.reshape(-1, 9), GOLD["blocks_enc"][-e.shape[0]:])


@pytest.mark.parametrize("M,K,ldx", [(1, 8, None), (17, 24, None), (600, 200, None), (300, 2560, 2600),
                                     (2048, 2560, None)])
def test_pack_act_ragged_shapes_against_oracle(zest_gpu, oracle, M, K, ldx):
    x = make_data(M * K, M * 31 + K).reshape(M, K)
    assert np.array_equal(gpu_pack(zest_gpu, x, ldx), oracle.encode_rows(x))


def test_pack_act_padding_is_zero(zest_gpu):
    import torch
    M, K = 70, 72  # rows pad to 256, columns to 128
    x = torch.from_numpy(make_data(M * K, 5).reshape(M, K)).cuda()
    out = torch.full((zest_gpu.bfp16_bytes(M, K),), 0xAB, dtype=torch.uint8, device="cuda")
    zest_gpu.pack_act(x, out)
    torch.cuda.synchronize()
    full = zest_gpu.tiles_to_blocks(out.cpu().numpy(), zest_gpu.rows_pad(M), zest_gpu.k_pad(K))
    assert not full[M:].any() and not full[:, K // 8:].any()


def test_pack_act_outlier_channels_full_size(zest_gpu, oracle):
    # BASELINE config 2's activations: N(0,1) with 1% of channels x20
    M, K = 2048, 2560
    rng = Rng(2)
    x = rng.normal(M * K).reshape(M, K)
    ch = rng.ints(K // 100, 0, K - 1)
    x[:, ch] *= 20.0
    assert np.array_equal(gpu_pack(zest_gpu, x), oracle.encode_rows(x))


# ---- the expanded activation operand (the GEMM's A) ----------------------

def gpu_pack_x(z, x: np.ndarray, ldx: int | None = None):
    """(pack_act_x bytes, expand_act(pack_act) bytes) of x, as numpy."""
    import torch
    m, k = x.shape
    if ldx is None:
        xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    else:
        full = torch.zeros((m, ldx), dtype=torch.float32)
        full[:, :k] = torch.from_numpy(x)
        xt = full.cuda()[:, :k]
    direct = torch.full((z.act_bytes(m, k),), 0xAB, dtype=torch.uint8, device="cuda")
    z.pack_act_x(xt, direct)
    via = z.expand_act(z.pack_act(xt), m, k)
    torch.cuda.synchronize()
    return direct.cpu().numpy(), via.cpu().numpy()


@pytest.mark.parametrize("M,K,ldx", [(1, 8, None), (17, 24, None), (600, 200, None), (300, 2560, 2600),
                                     (2048, 2560, None), (70, 72, None)])
def test_pack_act_x_is_the_decoded_pack(zest_gpu, oracle, M, K, ldx):
    # the expanded operand holds exactly the values the bfp16 bytes stand for:
    # byte-equal to expanding zest_pack_act's output (padding included), and
    # value-equal (bitwise) to the oracle's encode -> decode
    x = make_data(M * K, M * 17 + K).reshape(M, K)
    direct, via = gpu_pack_x(zest_gpu, x, ldx)
    assert np.array_equal(direct, via)
    got = zest_gpu.expanded_to_rows(direct, M, K)
    assert np.array_equal(got.view(np.uint32), oracle.decode_rows(oracle.encode_rows(x)).view(np.uint32))
    full = zest_gpu.expanded_to_rows(direct, zest_gpu.rows_pad(M), zest_gpu.k_pad(K))
    assert not full[M:].any() and not full[:, K:].any()


def test_pack_act_x_golden_and_edge_blocks(zest_gpu, oracle):
    # zero, subnormal, tiny, saturating and near-FLT_MAX blocks take the
    # general expansion; their decoded values must still be exact
    x = GOLD["blocks_x"]
    n = x.shape[0] // 64 * 64
    for rows in (x[:n].reshape(-1, 64), edge_blocks().reshape(1, -1)):
        direct, via = gpu_pack_x(zest_gpu, rows)
        assert np.array_equal(direct, via)
        got = zest_gpu.expanded_to_rows(direct, *rows.shape)
        assert np.array_equal(got.view(np.uint32), oracle.decode_rows(oracle.encode_rows(rows)).view(np.uint32))


def gpu_convert(z, wtype: int, raw: np.ndarray, n: int, k: int) -> np.ndarray:
    import torch
    rt = torch.from_numpy(np.ascontiguousarray(raw)).cuda()
    out = z.convert_weight(wtype, rt, n, k)
    torch.cuda.synchronize()
    return z.tiles_to_blocks(out.cpu().numpy(), n, k)


@pytest.mark.parametrize("wtype,N,K", [(8, 256, 512), (8, 300, 2560), (8, 100, 96), (12, 256, 512),
                                       (12, 333, 2560), (12, 9728, 2560), (12, 2560, 9728), (8, 2560, 4096)])
def test_convert_weight_matches_oracle(zest_gpu, oracle, wtype, N, K):
    import torch
    quant = load_quant()
    w = Rng(N + K + wtype).normal(N * K, 0.0, 0.02).reshape(N, K)
    raw = quant.quantize(wtype, torch.from_numpy(w)).numpy()
    want = oracle.encode_rows(oracle.dequant(wtype, raw, N, K))
    assert np.array_equal(gpu_convert(zest_gpu, wtype, raw, N, K), want)


def test_convert_weight_npu_order_matches_reference_golden(zest_gpu):
    # F32 weights through the converter land, via the bijection, exactly on
    # the reference packer's bfp16_pack_b bytes
    for N, K, n, k, cols in [(1024, 256, 64, 64, 8), (512, 128, 32, 64, 4)]:
        w = make_data(N * K, 7 + N + K).reshape(N, K)
        got = to_npu_order(gpu_convert(zest_gpu, 0, w.view(np.uint8), N, K), b_block_index(N, K, n, k, cols))
        assert np.array_equal(got, GOLD[f"b_{N}x{K}_n{n}k{k}c{cols}"])


def test_convert_extreme_quant_blocks(zest_gpu, oracle):
    # Q8_0 blocks with d = 0, the largest fp16 d, subnormal d and +-128 quants
    rng = Rng(9)
    n, k = 16, 256
    raw = rng.ints(n * k // 32 * 34, 0, 255).astype(np.uint8).reshape(n, k // 32, 34)
    ds = np.array([0.0, 65504.0, 6e-8, -1.0, 2.0 ** -14, 1e-3, -3e-5, 1.0], dtype=np.float16)
    raw[:, :, :2] = ds[rng.ints(n * k // 32, 0, 7)].view(np.uint8).reshape(n, k // 32, 2)
    raw = raw.reshape(n, -1)
    want = oracle.encode_rows(oracle.dequant(8, raw, n, k))
    assert np.array_equal(gpu_convert(zest_gpu, 8, raw, n, k), want)


# ---- every GGUF weight type --------------------------------------------------------
# The reference converts any type ggml dequantises (src/ggml-zest.cpp:1066-1072);
# its test covers f16, q4_0 and q6_K beside q8_0 and q4_K (tests/test-mul-mat.cpp:
# 140-156). Byte-exact against the oracle's dequantisation + encoder, on
# quantised normal weights and on random bytes (every code, bit and scale).

GGUF = {"f16": 1, "bf16": 30, "q4_0": 2, "q4_1": 3, "q5_0": 6, "q5_1": 7, "q8_0": 8,
        "q2_K": 10, "q3_K": 11, "q4_K": 12, "q5_K": 13, "q6_K": 14, "iq4_nl": 20, "iq4_xs": 23}
K_QUANTS = {10, 11, 12, 13, 14, 23}  # 256-value super-blocks
# byte ranges of each block's fp16 fields (kept finite in the random blocks)
F16_FIELDS = {2: [(0, 2)], 3: [(0, 4)], 6: [(0, 2)], 7: [(0, 4)], 8: [(0, 2)], 10: [(80, 84)],
              11: [(108, 110)], 12: [(0, 4)], 13: [(0, 4)], 14: [(208, 210)], 20: [(0, 2)], 23: [(0, 2)]}


def random_gguf(oracle, wtype: int, n: int, k: int, seed: int) -> np.ndarray:
    """n rows of random GGUF bytes whose fp16 (bf16) fields are finite."""
    rng = np.random.default_rng(seed)
    rb = oracle.row_bytes(wtype, k)
    raw = rng.integers(0, 256, (n, rb), dtype=np.uint8)
    if wtype in (1, 30):
        v = raw.view(np.uint16)
        exp_mask, top = (0x7C00, 0x4000) if wtype == 1 else (0x7F80, 0x4000)
        v[(v & exp_mask) == exp_mask] &= np.uint16(~top & 0xFFFF)
        return raw
    blk = 256 if wtype in K_QUANTS else 32
    bb = rb // (k // blk)
    b = raw.reshape(n, k // blk, bb)
    for lo, hi in F16_FIELDS[wtype]:
        h = rng.normal(0, 1, (n, k // blk, (hi - lo) // 2)) * np.exp2(rng.integers(-20, 8, (n, k // blk, (hi - lo) // 2)))
        b[:, :, lo:hi] = h.astype(np.float16).view(np.uint8).reshape(n, k // blk, hi - lo)
    return raw


def _shapes(wtype):
    if wtype in K_QUANTS:
        return [(256, 512), (300, 2560), (37, 256)]
    if wtype in (1, 30):
        return [(256, 512), (300, 2560), (37, 200)]  # K % 64 == 8
    return [(256, 512), (300, 2560), (37, 96)]  # K % 64 == 32: half a tile column of padding


@pytest.mark.parametrize("name", list(GGUF))
def test_convert_every_type_matches_oracle(zest_gpu, oracle, name):
    wtype = GGUF[name]
    for i, (N, K) in enumerate(_shapes(wtype)):
        w = Rng(N + K + wtype).normal(N * K, 0.0, 0.02).reshape(N, K)
        raw = oracle.quantize(wtype, w)
        want = oracle.encode_rows(oracle.dequant(wtype, raw, N, K))
        assert np.array_equal(gpu_convert(zest_gpu, wtype, raw, N, K), want), (name, N, K)
        raw = random_gguf(oracle, wtype, N, K, seed=wtype * 100 + i)
        want = oracle.encode_rows(oracle.dequant(wtype, raw, N, K))
        assert np.array_equal(gpu_convert(zest_gpu, wtype, raw, N, K), want), (name, N, K, "random")


@pytest.mark.parametrize("name", ["q4_0", "q5_1", "q3_K", "q6_K", "f16", "iq4_xs"])
def test_convert_gu_every_type_is_the_interleaved_pair(zest_gpu, oracle, name):
    import torch
    wtype, F, K = GGUF[name], 96, 512
    gate, up = (torch.from_numpy(random_gguf(oracle, wtype, F, K, seed=s)).cuda() for s in (1, 2))
    pair = zest_gpu.convert_weight_gu(wtype, gate, up, F, K).cpu().numpy()
    bg = zest_gpu.tiles_to_blocks(zest_gpu.convert_weight(wtype, gate, F, K).cpu().numpy(), F, K)
    bu = zest_gpu.tiles_to_blocks(zest_gpu.convert_weight(wtype, up, F, K).cpu().numpy(), F, K)
    bp = zest_gpu.tiles_to_blocks(pair, zest_gpu.rows_pad(2 * F), K)
    r = np.arange(F)
    dst = (r // 32) * 64 + r % 32
    assert np.array_equal(bp[dst], bg) and np.array_equal(bp[dst + 32], bu)


@pytest.mark.parametrize("name", ["q8_0", "q4_0", "q5_0", "q3_K", "q6_K", "iq4_nl"])
def test_convert_two_byte_aligned_rows(zest_gpu, oracle, name):
    # the types whose rows need only 2-byte alignment, from a buffer that
    # starts 2 bytes past a 4-byte boundary: the converter's aligned loads
    # then start before the buffer (inside the allocation) and must neither
    # read past its end nor take bytes of the neighbouring block
    import torch
    wtype = GGUF[name]
    for N, K in ([(37, 96), (5, 32)] if wtype not in K_QUANTS else [(37, 256)]):
        raw = random_gguf(oracle, wtype, N, K, seed=wtype + N)
        want = oracle.encode_rows(oracle.dequant(wtype, raw, N, K))
        buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device="cuda")
        buf[2:2 + raw.size] = torch.from_numpy(raw.reshape(-1)).cuda()
        out = zest_gpu.convert_weight(wtype, buf[2:2 + raw.size], N, K)
        torch.cuda.synchronize()
        assert np.array_equal(zest_gpu.tiles_to_blocks(out.cpu().numpy(), N, K), want), (name, N, K)


def test_convert_rejects_bad_rows(zest_gpu, oracle):
    import torch
    raw = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError):
        zest_gpu.convert_weight(3, raw[2:], 16, 256)     # Q4_1 rows need 4-byte alignment
    with pytest.raises(RuntimeError):
        zest_gpu.convert_weight(13, raw[4:], 16, 256)    # Q5_K rows need 16
    with pytest.raises(RuntimeError):
        zest_gpu.convert_weight(14, raw, 4, 128)         # Q6_K: K % 256 != 0
    with pytest.raises(RuntimeError):
        zest_gpu.convert_weight(23, raw[4:], 16, 256)    # IQ4_XS rows need 8
    with pytest.raises(RuntimeError):
        zest_gpu.convert_weight(2, raw, 4, 48)           # Q4_0: K % 32 != 0
    with pytest.raises(RuntimeError):
        zest_gpu.convert_weight(15, raw, 4, 256)         # Q8_K: no converter
    torch.cuda.synchronize()


def test_convert_blocks_at_the_exponent_edges(zest_gpu, oracle):
    # blocks whose largest exponent field is 0..12 (subnormals next to the
    # smallest normals) or 240..254, with the other seven values anywhere
    # below it, including values that round to +-128 and saturate
    rng = np.random.default_rng(12)
    n, k = 64, 512
    nb = n * k // 8
    top = np.concatenate([np.arange(0, 13), np.arange(240, 255)])
    e = top[rng.integers(0, len(top), nb)]
    lead = ((e.astype(np.uint32) << 23) | rng.integers(0, 1 << 23, nb).astype(np.uint32)
            | (rng.integers(0, 2, nb).astype(np.uint32) << 31))
    rest_e = np.maximum(e[:, None] - rng.integers(0, 30, (nb, 7)), 0).astype(np.uint32)
    rest = ((rest_e << 23) | rng.integers(0, 1 << 23, (nb, 7)).astype(np.uint32)
            | (rng.integers(0, 2, (nb, 7)).astype(np.uint32) << 31))
    # some blocks: a value just under the top of the binade (rounds to 128)
    near = rng.random(nb) < 0.2
    lead[near] = (lead[near] & np.uint32(0xFF800000)) | np.uint32(0x7FFFFF)
    blocks = np.concatenate([lead[:, None], rest], axis=1)
    perm = rng.permuted(np.tile(np.arange(8), (nb, 1)), axis=1)
    blocks = np.take_along_axis(blocks, perm, axis=1)
    w = blocks.reshape(n, k).view(np.float32)
    want = oracle.encode_rows(w)
    assert np.array_equal(gpu_convert(zest_gpu, 0, w.view(np.uint8), n, k), want)
    # the same values through a 16-bit type's path (BF16 keeps the exponent)
    bf = (w.view(np.uint32) >> 16).astype(np.uint16)
    want = oracle.encode_rows(oracle.dequant(30, bf.view(np.uint8), n, k))
    assert np.array_equal(gpu_convert(zest_gpu, 30, bf.view(np.uint8), n, k), want)


def test_convert_random_shapes_into_garbage_buffers(zest_gpu, oracle):
    # a seeded sweep: every type at random row counts and widths, quantised
    # weights and random bytes, each converted into a zero-filled and a
    # garbage-filled buffer; the values match the oracle and the padding
    # comes out the same in both (the converter writes every byte it owns),
    # and so does the gate/up pair's
    import torch
    rng = np.random.default_rng(5)
    names = list(GGUF)
    for case in range(2 * len(names)):
        name = names[case % len(names)]
        wtype = GGUF[name]
        blk = 256 if wtype in K_QUANTS else (8 if wtype in (1, 30) else 32)
        N = int(rng.choice([1, 15, 17, 31, 32, 33, 255, 257, 1000]))
        K = int(rng.integers(1, 24)) * blk * int(rng.choice([1, 2]))
        if rng.random() < 0.5:
            raw = random_gguf(oracle, wtype, N, K, seed=500 + case)
        else:
            raw = oracle.quantize(wtype, rng.normal(0, 0.02, (N, K)).astype(np.float32))
        want = oracle.encode_rows(oracle.dequant(wtype, raw, N, K))
        rt = torch.from_numpy(np.ascontiguousarray(raw)).cuda()
        zero = zest_gpu.empty_packed(N, K)
        zero.zero_()
        junk = torch.full_like(zero, 0xA5)
        zest_gpu.convert_weight(wtype, rt, N, K, out=zero)
        zest_gpu.convert_weight(wtype, rt, N, K, out=junk)
        torch.cuda.synchronize()
        assert np.array_equal(zest_gpu.tiles_to_blocks(zero.cpu().numpy(), N, K), want), (name, N, K)
        assert torch.equal(zero, junk), (name, N, K, int((zero != junk).sum()))
        if N % 32 == 0:
            up = torch.from_numpy(random_gguf(oracle, wtype, N, K, seed=900 + case)).cuda()
            pz = torch.zeros(zest_gpu.bfp16_bytes(2 * N, K), dtype=torch.uint8, device="cuda")
            pj = torch.full_like(pz, 0x5A)
            zest_gpu.convert_weight_gu(wtype, rt, up, N, K, out=pz)
            zest_gpu.convert_weight_gu(wtype, rt, up, N, K, out=pj)
            torch.cuda.synchronize()
            assert torch.equal(pz, pj), (name, "gu", N, K)
