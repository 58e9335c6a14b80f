"""The CPU oracle pinned against the reference's golden vectors, its known
answer tests, closed forms and brute force (no GPU). Mirrors
tests/test-bfp16-pack.cpp and the accuracy contract of tests/test-mul-mat.cpp."""
from __future__ import annotations

import hashlib

import numpy as np
import pytest
from gen import Rng, make_data
from helpers import GOLDEN, RefPacker, gemm_check, load_quant, nrmse

GOLD = np.load(GOLDEN / "bfp16_golden.npz")

A_SHAPES = [(512, 256, 128, 64), (256, 384, 64, 128), (1024, 6144, 128, 64)]
B_SHAPES = [(1024, 256, 64, 64, 8), (4096, 2048, 64, 64, 8), (2048, 6144, 64, 128, 8), (512, 128, 32, 64, 4)]


def test_encode_matches_reference_golden_blocks(oracle):
    got = oracle.encode_rows(GOLD["blocks_x"]).reshape(-1, 9)
    assert np.array_equal(got, GOLD["blocks_enc"])


def test_saturation_kat(oracle):
    # tests/test-bfp16-pack.cpp:168-175
    blk = np.ldexp(np.array([127.75, 1.0, -3.5, 0.0, 64.0, -127.5, 0.25, 100.5], dtype=np.float32), -6)
    enc = oracle.encode_rows(blk[None, :])[0, 0]
    m = enc[1:].view(np.int8)
    assert enc[0] == 127 and m[0] == 127 and m[5] == -128 and m[7] == 100


def test_zero_block_is_all_zero_bytes(oracle):
    z = np.array([[0.0, -0.0, 0.0, 0.0, -0.0, 0.0, 0.0, 0.0]], dtype=np.float32)
    assert not oracle.encode_rows(z).any()


def test_decode_every_exponent_byte(oracle):
    # tests/test-bfp16-pack.cpp:180-191: every exponent byte, mantissas -128..127
    e = np.repeat(np.arange(256, dtype=np.uint8), 32)
    m = np.tile(np.arange(-128, 128, dtype=np.int8), 256).reshape(-1, 8)
    blocks = np.concatenate([e[:, None], m.view(np.uint8)], axis=1)
    got = oracle.decode_rows(blocks[:, None, :]).reshape(-1, 8)
    with np.errstate(over="ignore"):  # 128 * 2^122 overflows to -inf in float, as in the reference
        want = np.ldexp(m.astype(np.float64), e[:, None].astype(np.int32) - 133).astype(np.float32)
    assert np.array_equal(got, want)


def test_encode_decode_round_trip_is_exact_for_representable_blocks(oracle):
    # a block whose largest mantissa magnitude is in 64..127 re-encodes to
    # itself: the exponent byte is recovered and every value is exact
    # (-128 is left out: its float exponent is one above the block's)
    rng = Rng(5)
    n = 4096
    e = rng.ints(n, 8, 250).astype(np.uint8)
    m = rng.ints(n * 8, -127, 127).astype(np.int8).reshape(n, 8)
    m[:, 0] = np.array([127, -127, 64, -64], dtype=np.int8)[rng.ints(n, 0, 3)]
    blocks = np.concatenate([e[:, None], m.view(np.uint8)], axis=1)
    x = oracle.decode_rows(blocks[:, None, :])
    assert np.array_equal(oracle.encode_rows(x).reshape(n, 9), blocks)


def test_encoder_matches_independent_float64_statement(oracle):
    # the test's own reference encoder (tests/test-bfp16-pack.cpp:21-38) works
    # in double; restate it with numpy float64 and compare on wide data
    x = make_data(64 * 1024, 99).reshape(-1, 8)
    bits = x.view(np.uint32)
    e = ((bits >> 23) & 0xFF).max(axis=1)
    q = np.rint(np.ldexp(x.astype(np.float64), (133 - e.astype(np.int32))[:, None]))
    q = np.clip(q, -128, 127).astype(np.int8)
    want = np.concatenate([e.astype(np.uint8)[:, None], q.view(np.uint8)], axis=1)
    assert np.array_equal(oracle.encode_rows(x).reshape(-1, 9), want)


@pytest.mark.parametrize("M,K,m,k", A_SHAPES)
def test_pack_a_order_matches_reference(oracle, M, K, m, k):
    x = make_data(M * K, 1 + M + K).reshape(M, K)
    got = oracle.pack_a(x, m, k)
    key = f"a_{M}x{K}_m{m}k{k}"
    if key in GOLD:
        assert np.array_equal(got, GOLD[key])
    assert hashlib.sha256(got.tobytes()).digest() == GOLD[key + "_sha256"].tobytes()


@pytest.mark.parametrize("N,K,n,k,cols", B_SHAPES)
def test_pack_b_order_matches_reference(oracle, N, K, n, k, cols):
    w = make_data(N * K, 7 + N + K).reshape(N, K)
    got = oracle.pack_b(w, n, k, cols)
    key = f"b_{N}x{K}_n{n}k{k}c{cols}"
    if key in GOLD:
        assert np.array_equal(got, GOLD[key])
    assert hashlib.sha256(got.tobytes()).digest() == GOLD[key + "_sha256"].tobytes()


def test_oracle_against_reference_packer_built_here(oracle):
    try:
        ref = RefPacker("avx2")
    except FileNotFoundError:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    for seed in (3, 4):
        x = make_data(256 * 512, seed).reshape(256, 512)
        assert np.array_equal(oracle.pack_a(x, 128, 64), ref.pack_a(x, 128, 64))
        assert np.array_equal(oracle.pack_b(x, 64, 64, 4), ref.pack_b(x, 64, 64, 4))


# ---- GGUF dequant --------------------------------------------------------------

def _fp16(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


def test_q8_0_dequant_closed_form(oracle):
    q = np.arange(-128, 128, dtype=np.int8).reshape(8, 32)
    raw = np.concatenate([np.concatenate([_fp16(0.5 * (i + 1)), q[i].view(np.uint8)]) for i in range(8)])
    y = oracle.dequant(8, raw, 1, 256)
    want = (q.astype(np.float64) * (0.5 * (np.arange(8) + 1))[:, None]).reshape(-1)
    assert np.array_equal(y.reshape(-1), want.astype(np.float32))


def _q4k_block(d, dmin, sc, mn, q):
    """A Q4_K block from 8 (scale, min) pairs and 256 nibbles, packed by the
    inverse of the 6-bit layout (scales[0..3] = sc|hi2(sc4..7), [4..7] =
    m|hi2(m4..7), [8..11] = lo4(sc4..7)|lo4(m4..7)<<4)."""
    sc = np.asarray(sc, dtype=np.uint8)
    mn = np.asarray(mn, dtype=np.uint8)
    s = np.zeros(12, dtype=np.uint8)
    s[0:4] = sc[0:4] | ((sc[4:8] >> 4) << 6)
    s[4:8] = mn[0:4] | ((mn[4:8] >> 4) << 6)
    s[8:12] = (sc[4:8] & 0xF) | ((mn[4:8] & 0xF) << 4)
    q = np.asarray(q, dtype=np.uint8).reshape(8, 32)
    qs = (q[0::2] | (q[1::2] << 4)).reshape(-1)
    return np.concatenate([_fp16(d), _fp16(dmin), s, qs])


def test_q4_k_dequant_hand_built_blocks(oracle):
    # every sub-block gets its own scale and min, including the split 6-bit
    # fields of sub-blocks 4..7; constant nibbles per sub-block reveal the
    # order (low nibbles of a 32-byte run first, then the high nibbles)
    sc = [1, 2, 3, 63, 17, 33, 48, 62]
    mn = [0, 5, 63, 9, 21, 40, 63, 1]
    q = np.repeat(np.arange(8) + 3, 32)
    for d, dmin in ((0.25, 0.125), (1.5, 0.0078125)):
        raw = _q4k_block(d, dmin, sc, mn, q)
        y = oracle.dequant(12, raw, 1, 256).reshape(8, 32)
        want = np.array([d * sc[j] * (j + 3) - dmin * mn[j] for j in range(8)], dtype=np.float64)
        assert np.array_equal(y, np.repeat(want.astype(np.float32)[:, None], 32, axis=1))
    # varying nibbles inside one sub-block keep their positions
    qv = np.arange(256) % 16
    raw = _q4k_block(1.0, 0.0, [1] * 8, [0] * 8, qv)
    assert np.array_equal(oracle.dequant(12, raw, 1, 256).reshape(-1), qv.astype(np.float32))


@pytest.mark.parametrize("wtype", [8, 12])
def test_quantize_dequantize_round_trip_bound(oracle, wtype):
    import torch
    quant = load_quant()
    n, k = 64, 512
    w = Rng(17).normal(n * k, 0.0, 0.02).reshape(n, k)
    raw = quant.quantize(wtype, torch.from_numpy(w)).numpy()
    y = oracle.dequant(wtype, raw, n, k)
    if wtype == 8:
        step = np.abs(w.reshape(n, k // 32, 32)).max(axis=2) / 127.0
        err = np.abs(y - w).reshape(n, k // 32, 32).max(axis=2)
        # half a step, plus the fp16 rounding of d over |q| <= 127 steps
        assert (err <= (0.5 + 127 * 2.0 ** -11) * step + 1e-7).all()
    else:
        assert nrmse(y, w) < 0.08  # 4-bit: ~ (range/15)/sqrt(12) / std
        assert np.abs(y - w).max() < 0.02


# The rest of GGUF's weight types (the reference converts any type ggml can
# dequantise, src/ggml-zest.cpp:1066-1072; its own test covers f16, q4_0 and
# q6_K, tests/test-mul-mat.cpp:140-156). The builders below pack blocks from
# per-position codes, field by field in the order of the block structs, so
# that a value read from the wrong nibble, bit or scale shows up as a wrong
# value at a known position.

F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, BF16 = 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 30
IQ4_NL, IQ4_XS = 20, 23
ALL_TYPES = [0, F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS]


def _u32le(v):
    return np.array([v], dtype="<u4").view(np.uint8)


def _nibbles32(q):
    """32 codes of a 32-value block: value j in the low nibble of byte j,
    value j + 16 in the high nibble; and the fifth bits as a 32-bit word."""
    q = np.asarray(q, dtype=np.int64)
    qs = ((q[:16] & 0xF) | ((q[16:] & 0xF) << 4)).astype(np.uint8)
    qh = int(sum(int(q[j] >> 4 & 1) << j for j in range(32)))
    return qs, qh


def test_f16_bf16_every_bit_pattern(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    y = oracle.dequant(F16, bits.view(np.uint8), 1, 65536).reshape(-1)
    want = bits.view(np.float16).astype(np.float32)
    same = (y.view(np.uint32) == want.view(np.uint32)) | (np.isnan(y) & np.isnan(want))
    assert same.all()
    y = oracle.dequant(BF16, bits.view(np.uint8), 1, 65536).reshape(-1)
    assert np.array_equal(y.view(np.uint32), bits.astype(np.uint32) << 16)


def test_q4_0_q5_0_hand_built_blocks(oracle):
    rng = np.random.default_rng(3)
    for d in (0.5, 3.0e-4, -2.0):
        q4 = rng.integers(0, 16, 32)
        qs, _ = _nibbles32(q4)
        y = oracle.dequant(Q4_0, np.concatenate([_fp16(d), qs]), 1, 32).reshape(-1)
        assert np.array_equal(y, ((q4 - 8) * np.float64(np.float16(d))).astype(np.float32))
        q5 = rng.integers(0, 32, 32)
        qs, qh = _nibbles32(q5)
        y = oracle.dequant(Q5_0, np.concatenate([_fp16(d), _u32le(qh), qs]), 1, 32).reshape(-1)
        assert np.array_equal(y, ((q5 - 16) * np.float64(np.float16(d))).astype(np.float32))


def test_q4_1_q5_1_hand_built_blocks(oracle):
    rng = np.random.default_rng(4)
    for d, m in ((0.25, -1.75), (1.0e-3, 0.3), (2.0, 0.0)):
        dd, mm = np.float32(np.float16(d)), np.float32(np.float16(m))
        q4 = rng.integers(0, 16, 32)
        qs, _ = _nibbles32(q4)
        y = oracle.dequant(Q4_1, np.concatenate([_fp16(d), _fp16(m), qs]), 1, 32).reshape(-1)
        assert np.array_equal(y, q4.astype(np.float32) * dd + mm)  # d*q exact: one rounding
        q5 = rng.integers(0, 32, 32)
        qs, qh = _nibbles32(q5)
        y = oracle.dequant(Q5_1, np.concatenate([_fp16(d), _fp16(m), _u32le(qh), qs]), 1, 32).reshape(-1)
        assert np.array_equal(y, q5.astype(np.float32) * dd + mm)


def test_32_value_types_agree_where_their_fields_meet(oracle):
    # Q4_1 with m = -8d is Q4_0; Q5_1 with no fifth bits is Q4_1; Q5_0 with
    # every fifth bit set is Q4_1 with m = 0
    rng = np.random.default_rng(5)
    for _ in range(20):
        d = float(np.float16(rng.uniform(-4, 4)))
        qs = rng.integers(0, 256, 16).astype(np.uint8)
        a = oracle.dequant(Q4_0, np.concatenate([_fp16(d), qs]), 1, 32)
        b = oracle.dequant(Q4_1, np.concatenate([_fp16(d), _fp16(-8 * d), qs]), 1, 32)
        assert np.array_equal(a, b)
        m = float(np.float16(rng.uniform(-1, 1)))
        c = oracle.dequant(Q4_1, np.concatenate([_fp16(d), _fp16(m), qs]), 1, 32)
        e = oracle.dequant(Q5_1, np.concatenate([_fp16(d), _fp16(m), _u32le(0), qs]), 1, 32)
        assert np.array_equal(c, e)
        f = oracle.dequant(Q5_0, np.concatenate([_fp16(d), _u32le(0xFFFFFFFF), qs]), 1, 32)
        g = oracle.dequant(Q4_1, np.concatenate([_fp16(d), _fp16(0.0), qs]), 1, 32)
        assert np.array_equal(f, g)


def _q2k_block(d, dmin, sc, mn, q):
    """256 two-bit codes; 16 (scale, min) nibble pairs. Half h, group g of 16:
    codes at bits 2(g//2) of qs[32h + 16(g%2) + l], scale byte 8h + g."""
    q = np.asarray(q, dtype=np.int64).reshape(2, 8, 16)
    qs = np.zeros((2, 32), dtype=np.int64)
    for h in range(2):
        for g in range(8):
            qs[h, 16 * (g % 2):16 * (g % 2) + 16] |= q[h, g] << (2 * (g // 2))
    scales = (np.asarray(sc) | (np.asarray(mn) << 4)).astype(np.uint8)
    return np.concatenate([scales, qs.reshape(-1).astype(np.uint8), _fp16(d), _fp16(dmin)])


def _q3k_block(d, s6, q):
    """256 codes in -4..3 and 16 signed scales in -32..31."""
    q = np.asarray(q, dtype=np.int64).reshape(2, 8, 16)
    u = np.asarray(s6, dtype=np.int64) + 32
    sc = np.zeros(12, dtype=np.int64)
    for i in range(16):
        sc[i % 8] |= (u[i] & 0xF) << (0 if i < 8 else 4)
        sc[8 + i % 4] |= (u[i] >> 4) << (2 * (i // 4))
    qs = np.zeros((2, 32), dtype=np.int64)
    hm = np.zeros(32, dtype=np.int64)
    for h in range(2):
        for g in range(8):
            o = 16 * (g % 2)
            qs[h, o:o + 16] |= (q[h, g] & 3) << (2 * (g // 2))
            hm[o:o + 16] |= (q[h, g] >= 0).astype(np.int64) << (4 * h + g // 2)
    return np.concatenate([hm.astype(np.uint8), qs.reshape(-1).astype(np.uint8), sc.astype(np.uint8), _fp16(d)])


def _q5k_block(d, dmin, sc, mn, q):
    """Q4_K's header and nibbles, and the fifth bits of group j of 64 at bits
    2j (first 32) and 2j + 1 (second 32) of qh[l]."""
    q = np.asarray(q, dtype=np.int64).reshape(4, 2, 32)
    base = _q4k_block(d, dmin, sc, mn, (q & 0xF).reshape(-1))
    qh = np.zeros(32, dtype=np.int64)
    for j in range(4):
        qh |= (q[j, 0] >> 4) << (2 * j)
        qh |= (q[j, 1] >> 4) << (2 * j + 1)
    return np.concatenate([base[:16], qh.astype(np.uint8), base[16:]])


def _q6k_block(d, sc, q):
    """256 codes in -32..31, 16 int8 scales. Half h, quarter c of 32: value
    l's low 4 bits in nibble c//2 of ql[64h + 32(c%2) + l], high 2 bits at
    bits 2c of qh[32h + l]."""
    u = (np.asarray(q, dtype=np.int64) + 32).reshape(2, 4, 32)
    ql = np.zeros((2, 64), dtype=np.int64)
    qh = np.zeros((2, 32), dtype=np.int64)
    for h in range(2):
        for c in range(4):
            ql[h, 32 * (c % 2):32 * (c % 2) + 32] |= (u[h, c] & 0xF) << (4 * (c // 2))
            qh[h] |= (u[h, c] >> 4) << (2 * c)
    return np.concatenate([ql.reshape(-1).astype(np.uint8), qh.reshape(-1).astype(np.uint8),
                           np.asarray(sc, dtype=np.int8).view(np.uint8), _fp16(d)])


def test_q2_k_hand_built_blocks(oracle):
    rng = np.random.default_rng(6)
    q = rng.integers(0, 4, 256)
    sc, mn = rng.integers(0, 16, 16), rng.integers(0, 16, 16)
    d, dmin = np.float32(np.float16(0.0625)), np.float32(np.float16(0.01))
    y = oracle.dequant(Q2_K, _q2k_block(d, dmin, sc, mn, q), 1, 256).reshape(-1)
    g = np.arange(256) // 16
    want = (d * sc[g].astype(np.float32)) * q.astype(np.float32) - dmin * mn[g].astype(np.float32)
    assert np.array_equal(y, want)


def test_q3_k_hand_built_blocks_and_q2_k_relation(oracle):
    rng = np.random.default_rng(7)
    q = rng.integers(-4, 4, 256)
    s6 = rng.integers(-32, 32, 16)
    d = np.float32(np.float16(0.125))
    y = oracle.dequant(Q3_K, _q3k_block(d, s6, q), 1, 256).reshape(-1)
    g = np.arange(256) // 16
    assert np.array_equal(y, (d * s6[g].astype(np.float32)) * q.astype(np.float32))
    # with every hmask bit set the codes are Q2_K's 2-bit fields, and a scale
    # of 0..15 with min 0 is Q2_K's scale byte
    raw = _q3k_block(d, rng.integers(0, 16, 16), rng.integers(0, 4, 256))
    raw[:32] = 0xFF
    s = np.array([(raw[96 + i % 8] >> (0 if i < 8 else 4) & 0xF) | ((raw[104 + i % 4] >> (2 * (i // 4)) & 3) << 4)
                  for i in range(16)]) - 32
    q2 = np.concatenate([s.astype(np.uint8), raw[32:96], _fp16(d), _fp16(0.0)])
    assert np.array_equal(oracle.dequant(Q3_K, raw, 1, 256), oracle.dequant(Q2_K, q2, 1, 256))


def test_q5_k_hand_built_blocks_and_q4_k_relation(oracle):
    rng = np.random.default_rng(8)
    q = rng.integers(0, 32, 256)
    sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    d, dmin = np.float32(np.float16(0.03125)), np.float32(np.float16(0.0078125))
    y = oracle.dequant(Q5_K, _q5k_block(d, dmin, sc, mn, q), 1, 256).reshape(-1)
    g = np.arange(256) // 32
    assert np.array_equal(y, (d * sc[g].astype(np.float32)) * q.astype(np.float32) - dmin * mn[g].astype(np.float32))
    # with no fifth bits it is Q4_K over the same header and nibbles
    q4 = rng.integers(0, 16, 256)
    raw = _q5k_block(d, dmin, sc, mn, q4)
    assert not raw[16:48].any()
    assert np.array_equal(oracle.dequant(Q5_K, raw, 1, 256),
                          oracle.dequant(Q4_K, np.concatenate([raw[:16], raw[48:]]), 1, 256))


def test_q6_k_hand_built_blocks(oracle):
    rng = np.random.default_rng(9)
    q = rng.integers(-32, 32, 256)
    sc = rng.integers(-128, 128, 16)
    for d in (0.001, -0.5):
        dd = np.float32(np.float16(d))
        y = oracle.dequant(Q6_K, _q6k_block(d, sc, q), 1, 256).reshape(-1)
        g = np.arange(256) // 16
        assert np.array_equal(y, (dd * sc[g].astype(np.float32)) * q.astype(np.float32))
    # every position alone: one nonzero code walks the block
    for pos in (0, 15, 16, 31, 32, 63, 64, 95, 96, 127, 128, 191, 224, 255):
        qq = np.zeros(256, dtype=np.int64)
        qq[pos] = 31
        y = oracle.dequant(Q6_K, _q6k_block(1.0, np.ones(16), qq), 1, 256).reshape(-1)
        assert np.flatnonzero(y).tolist() == [pos] and y[pos] == 31.0


# IQ4_NL and IQ4_XS code into GGUF's published 16-level non-uniform grid
# (ggml-common.h kvalues_iq4nl; ggml itself is absent, so the grid is taken
# as published). IQ4_NL: d, qs[16]; IQ4_XS: d, scales_h, scales_l[4],
# qs[128] with a 6-bit scale per 32-value sub-block, dl = d*(ls - 32).
IQ4_GRID = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113])


def _iq4xs_block(d, ls, q):
    """One IQ4_XS super-block from d, 8 six-bit scales and 256 codes."""
    ls = np.asarray(ls, dtype=np.int64)
    sh = sum(int(ls[s] >> 4) << (2 * s) for s in range(8))
    sl = np.array([(ls[2 * i] & 0xF) | ((ls[2 * i + 1] & 0xF) << 4) for i in range(4)], dtype=np.uint8)
    qs = np.concatenate([_nibbles32(q[32 * s:32 * s + 32])[0] for s in range(8)])
    return np.concatenate([_fp16(d), np.array([sh], dtype="<u2").view(np.uint8), sl, qs])


def test_iq4_nl_hand_built_blocks(oracle):
    rng = np.random.default_rng(11)
    for d in (0.5, 3.0e-4, -2.0):
        q = rng.integers(0, 16, 32)
        qs, _ = _nibbles32(q)
        y = oracle.dequant(IQ4_NL, np.concatenate([_fp16(d), qs]), 1, 32).reshape(-1)
        assert np.array_equal(y, (IQ4_GRID[q] * np.float64(np.float16(d))).astype(np.float32))
    # each code once, in order, then reversed: the grid's own order
    q = np.concatenate([np.arange(16), np.arange(16)[::-1]])
    y = oracle.dequant(IQ4_NL, np.concatenate([_fp16(1.0), _nibbles32(q)[0]]), 1, 32).reshape(-1)
    assert y[:16].tolist() == IQ4_GRID.tolist() and y[16:].tolist() == IQ4_GRID[::-1].tolist()


def test_iq4_xs_hand_built_blocks(oracle):
    rng = np.random.default_rng(12)
    g = np.arange(256) // 32
    for d in (0.01, -1.5):
        ls, q = rng.integers(0, 64, 8), rng.integers(0, 16, 256)
        y = oracle.dequant(IQ4_XS, _iq4xs_block(d, ls, q), 1, 256).reshape(-1)
        dl = np.float32(np.float16(d)) * (ls - 32).astype(np.float32)
        assert np.array_equal(y, dl[g] * IQ4_GRID[q].astype(np.float32))
    # each sub-block's scale alone: scale 63 in sub-block s, 32 (dl = 0) elsewhere
    q = rng.integers(0, 16, 256)
    for s in range(8):
        ls = np.full(8, 32)
        ls[s] = 63
        y = oracle.dequant(IQ4_XS, _iq4xs_block(1.0, ls, q), 1, 256).reshape(-1)
        assert not y[g != s].any() and np.array_equal(y[g == s], 31.0 * IQ4_GRID[q[g == s]])
    # with every scale 33 (dl = d) a super-block is eight IQ4_NL blocks
    d = 0.0625
    nl = np.concatenate([np.concatenate([_fp16(d), _nibbles32(q[32 * s:32 * s + 32])[0]]) for s in range(8)])
    assert np.array_equal(oracle.dequant(IQ4_XS, _iq4xs_block(d, np.full(8, 33), q), 1, 256),
                          oracle.dequant(IQ4_NL, nl, 1, 256))


@pytest.mark.parametrize("wtype,bound", [
    (F16, 5e-4), (BF16, 4e-3), (Q4_0, 0.1), (Q4_1, 0.09), (Q5_0, 0.05), (Q5_1, 0.045), (Q8_0, 0.006),
    (Q2_K, 0.45), (Q3_K, 0.2), (Q4_K, 0.09), (Q5_K, 0.045), (Q6_K, 0.025), (IQ4_NL, 0.1), (IQ4_XS, 0.1)])
def test_oracle_quantiser_round_trip(oracle, wtype, bound):
    # the synthetic rows decode to the weights they came from, within the
    # type's resolution (nrmse over normal weights)
    n, k = 32, 512
    w = Rng(41 + wtype).normal(n * k, 0.0, 0.02).reshape(n, k)
    raw = oracle.quantize(wtype, w)
    assert raw.shape == (n, oracle.row_bytes(wtype, k))
    assert nrmse(oracle.dequant(wtype, raw, n, k), w) < bound


# ---- the reference matmul --------------------------------------------------------

def test_ref_mul_mat_integer_kat(oracle):
    # npu_self_test's operands (src/xdna-npu.cpp:142-156): exact under any order
    a, w = oracle.self_test_inputs(512, 128, 512)
    want = a.astype(np.int64) @ w.astype(np.int64).T
    got = oracle.mul_mat_f32(w, a)
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("wtype", [8, 12])
def test_ref_mul_mat_dequantises_then_dots(oracle, wtype):
    import torch
    quant = load_quant()
    n, k, m = 48, 512, 40
    w = Rng(23).normal(n * k, 0.0, 0.02).reshape(n, k)
    raw = quant.quantize(wtype, torch.from_numpy(w)).numpy()
    x = Rng(24).normal(m * k).reshape(m, k)
    y = oracle.ref_mul_mat(wtype, raw, n, k, x, threads=3)
    assert np.array_equal(y, oracle.mul_mat_f32(oracle.dequant(wtype, raw, n, k), x, threads=5))
    r64, ab = oracle.mul_mat_f64(oracle.dequant(wtype, raw, n, k), x)
    worst, _ = gemm_check(y, r64, ab, k)
    assert worst <= 1.0


def test_fp64_reference_against_numpy(oracle):
    w = Rng(31).normal(33 * 200).reshape(33, 200)
    x = Rng(32).normal(21 * 200).reshape(21, 200)
    r64, ab = oracle.mul_mat_f64(w, x, threads=4)
    assert np.allclose(r64, x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-12, atol=1e-12)
    assert np.allclose(ab, np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T, rtol=1e-12)


# ---- host ops ------------------------------------------------------------------

def test_rms_norm_closed_form_and_fp64(oracle):
    x = np.full((3, 256), 2.0, dtype=np.float32)
    y = oracle.rms_norm(x, 0.0)
    assert np.allclose(y, 1.0, rtol=0, atol=1e-6)
    x = Rng(41).normal(8 * 256, 0, 1.5).reshape(8, 256)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6)
    assert nrmse(oracle.rms_norm(x, 1e-6), want) < 1e-6


def test_glu_kinds_against_library_functions(oracle):
    from scipy.special import erf, expit
    g = Rng(43).normal(8 * 256, 0, 1.5).reshape(8, 256).astype(np.float32)
    u = Rng(44).normal(8 * 256, 0, 1.5).reshape(8, 256).astype(np.float32)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    assert nrmse(oracle.glu(2, g, u), g64 * expit(g64) * u64) < 1e-6                       # SwiGLU
    assert nrmse(oracle.glu(3, g, u), 0.5 * g64 * (1 + erf(g64 / np.sqrt(2))) * u64) < 1e-6  # GeGLU (erf)
    assert nrmse(oracle.glu(1, g, u), 0.5 * g64 * (1 + erf(g64 / np.sqrt(2))) * u64) < 2e-3  # tanh approximation
    assert nrmse(oracle.glu(4, g, u), g64 * expit(1.702 * g64) * u64) < 1e-6                 # quick GELU
    assert nrmse(oracle.glu(0, g, u), np.maximum(g64, 0) * u64) < 1e-7                       # ReGLU


def test_elementwise_ops(oracle):
    x = Rng(45).normal(4 * 64).reshape(4, 64)
    w = Rng(46).normal(64)
    assert np.array_equal(oracle.mul_row(x, w), x * w[None, :])
    assert np.array_equal(oracle.add_row(x, w), x + w[None, :])
    assert np.array_equal(oracle.add(x, x[::-1].copy()), x + x[::-1])
    assert np.array_equal(oracle.scale(x, np.float32(0.37), np.float32(0.25)),
                          x * np.float32(0.37) + np.float32(0.25))


@pytest.mark.parametrize("mode", [0, 2])
def test_rope_is_a_rotation_by_pos_times_theta(oracle, mode):
    # no YaRN, no factors, attn_factor 1: each pair turns by pos*base^(-2p/n)
    T, H, D = 4, 3, 64
    x = Rng(47).normal(T * H * D).reshape(T, H, D)
    pos = np.array([0, 1, 17, 5000], dtype=np.int32)
    for n_dims in (D, D // 2):
        y = oracle.rope(x, pos, None, n_dims, mode, 0, 10000.0, 1.0, 0.0, 1.0, 32.0, 1.0)
        half = n_dims // 2
        p = np.arange(half)
        theta = pos[:, None].astype(np.float64) * 10000.0 ** (-2.0 * p / n_dims)[None, :]
        i0 = p if mode == 2 else 2 * p
        i1 = i0 + (half if mode == 2 else 1)
        z = (x[:, :, i0] + 1j * x[:, :, i1]) * np.exp(1j * theta)[:, None, :]
        assert np.allclose(y[:, :, i0], z.real, atol=2e-3)
        assert np.allclose(y[:, :, i1], z.imag, atol=2e-3)
        assert np.array_equal(y[:, :, n_dims:], x[:, :, n_dims:])
        assert np.array_equal(y[0], x[0])  # position 0 turns nothing


def test_rope_yarn_corr_dims_closed_form(oracle):
    # YaRN's correction dims are where a rotation pair completes beta turns
    # over the original context: pair d turns n_ctx * base^(-2d/n) / (2 pi)
    # times. The first dim is the last pair (rounded down) turning at least
    # beta_fast times, the second the first pair (rounded up) turning at most
    # beta_slow times, both clamped to [0, n - 1]
    def turns(n, ctx, base, d):
        return ctx * base ** (-2.0 * d / n) / (2 * np.pi)

    checked = 0
    for n, ctx, base, bf, bs in [(64, 4096, 10000.0, 32.0, 1.0), (128, 2048, 500000.0, 32.0, 1.0),
                                 (96, 8192, 10000.0, 16.0, 2.0), (32, 512, 1e6, 64.0, 0.5)]:
        lo, hi = oracle.corr_dims(n, ctx, base, bf, bs)
        assert lo == int(lo) and hi == int(hi) and 0 <= lo <= hi <= n - 1
        if lo > 0:
            assert turns(n, ctx, base, lo) >= bf > turns(n, ctx, base, lo + 1)
            checked += 1
        else:
            assert turns(n, ctx, base, 0) <= bf * (1 + 1e-6) or turns(n, ctx, base, 1) < bf
        if hi < n - 1:
            assert turns(n, ctx, base, hi) <= bs < turns(n, ctx, base, hi - 1)
            checked += 1
    assert checked >= 4


def test_rope_yarn_ramp_ends_and_attention_scale(oracle):
    # With ext_factor 1 and frequency scale s, pairs up to the first
    # correction dim keep the extrapolated angle pos * base^(-2p/n), pairs from
    # the second on take the interpolated one s * pos * base^(-2p/n), the mix
    # between them moves linearly in the pair index, and every pair's
    # magnitude is attn_factor * (1 + 0.1 ln(1/s)) (YaRN's attention scaling)
    n, ctx, base, s, attn = 64, 4096, 10000.0, 0.25, 0.9
    lo, hi = (int(v) for v in oracle.corr_dims(n, ctx, base, 32.0, 1.0))
    pos = np.array([3], dtype=np.int32)
    x = np.zeros((1, 1, n), dtype=np.float32)
    x[0, 0, 0::2] = 1.0  # each pair (1, 0): the output is (m cos a, m sin a)
    y = oracle.rope(x, pos, None, n, 0, ctx, base, s, 1.0, attn, 32.0, 1.0)[0, 0]
    mag = np.hypot(y[0::2], y[1::2]).astype(np.float64)
    ang = np.arctan2(y[1::2], y[0::2]).astype(np.float64)
    assert np.allclose(mag, attn * (1 + 0.1 * np.log(1 / s)), rtol=1e-5)
    p = np.arange(n // 2)
    ext = 3.0 * base ** (-2.0 * p / n)
    wrap = lambda a: (a + np.pi) % (2 * np.pi) - np.pi
    assert np.allclose(wrap(ang[:lo + 1] - ext[:lo + 1]), 0, atol=2e-5)
    assert np.allclose(wrap(ang[hi:] - s * ext[hi:]), 0, atol=2e-5)
    # between the dims: the share of the extrapolated angle falls linearly
    mid = np.arange(lo + 1, hi)
    share = (ang[mid] - s * ext[mid]) / ((1 - s) * ext[mid])
    keep = ext[mid] > 1e-3  # where the angle resolves the share
    assert keep.sum() >= 5
    step = np.diff(share[keep]) / np.diff(mid[keep])
    assert np.allclose(step, -1.0 / (hi - lo), atol=2e-3) and np.all((share > -1e-3) & (share < 1 + 1e-3))
    # ext_factor 0: plain interpolation, magnitude attn_factor
    y0 = oracle.rope(x, pos, None, n, 0, ctx, base, s, 0.0, attn, 32.0, 1.0)[0, 0]
    assert np.allclose(np.hypot(y0[0::2], y0[1::2]), attn, rtol=1e-5)
    assert np.allclose(wrap(np.arctan2(y0[1::2], y0[0::2]) - s * ext), 0, atol=2e-5)