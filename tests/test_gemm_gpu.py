"""The HIP bfp16 GEMM against the oracle. Products of two bfp16 values are
exact in bf16 x bf16 -> fp32, so the only allowed difference from the
reference loop over the same decoded operands is fp32 summation order:
every output must sit inside |g - r64| <= 2 K 2^-24 sum|a b| (which any fp32
summation order of exact products keeps),
and the integer / exponent-shift known-answer tests must hold exactly."""
from __future__ import annotations

import numpy as np
import pytest
from gen import Rng, make_data, wide_blocks
from helpers import gemm_check, load_quant

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_gemm(z, x: np.ndarray, wtype: int, raw: np.ndarray, n: int):
    """The product path: x packed straight into the expanded operand, the
    weight converted into the bfp16 cache layout, then the GEMM."""
    import torch
    m, k = x.shape
    a = z.pack_act_x(_dev(x))
    w = z.convert_weight(wtype, _dev(raw), n, k)
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    c = z.gemm(a, m, w, n, k, nonfinite=nf)
    torch.cuda.synchronize()
    return c.cpu().numpy(), int(nf.item()), a, w


def decoded(z, oracle, packed, rows, k):
    """A packed bfp16 weight's values."""
    return oracle.decode_rows(z.tiles_to_blocks(packed.cpu().numpy(), rows, k))


def decoded_act(z, oracle, a, rows, k):
    """The expanded activation operand's values; they must be the oracle's
    bfp16 encoding, decoded (checked by the callers' data through
    test_pack_gpu, and here on every call)."""
    return z.expanded_to_rows(a.cpu().numpy(), rows, k)


def test_self_test_entry_point(zest_gpu):
    zest_gpu.self_test()


def test_integer_kat_exact(zest_gpu, oracle):
    # npu_self_test (src/xdna-npu.cpp:142-184) at several sizes
    for m, k, n in [(512, 128, 512), (1024, 2560, 768), (37, 64, 300)]:
        a, w = oracle.self_test_inputs(m, k, n)
        c, nf, _, _ = run_gemm(zest_gpu, a, 0, w.view(np.uint8), n)
        want = a.astype(np.int64) @ w.astype(np.int64).T
        assert np.array_equal(c, want.astype(np.float32)), (m, k, n)
        assert nf == 0


def test_exponent_shift_kat(zest_gpu, oracle):
    # raising every weight exponent byte by d scales every output by exactly
    # 2^d (tools/npu-ceiling-repro.cpp:14-23)
    import torch
    m, k, n = 256, 512, 512
    x = Rng(3).normal(m * k).reshape(m, k)
    w = Rng(4).normal(n * k, 0, 0.02).reshape(n, k)
    c0, _, a, wp = run_gemm(zest_gpu, x, 0, w.view(np.uint8), n)
    tiles = wp.view(-1, 1152)
    for d in (3, -5):
        shifted = wp.clone().view(-1, 1152)
        e = shifted[:, 1024:].to(torch.int32)
        shifted[:, 1024:] = torch.where(e > 0, e + d, e).to(torch.uint8)
        c = zest_gpu.gemm(a, m, shifted.view(-1), n, k)
        torch.cuda.synchronize()
        assert np.array_equal(c.cpu().numpy(), np.ldexp(c0, d))
    assert tiles.shape[0] > 0


@pytest.mark.parametrize("wtype,M,N,K", [
    (8, 1024, 2560, 2560),   # BASELINE config 1 (test-mul-mat shape), Q8_0
    (12, 600, 896, 1536),    # padded widths and a ragged batch (test-mul-mat.cpp:153-156)
    (12, 520, 8960, 1536),
    (0, 300, 200, 200),      # K not a multiple of 64
    (8, 1, 256, 512),
    (12, 2048, 1024, 2560),  # K/V projection of config 3
    (8, 1024, 1024, 4096),   # 64x64 tiles, one a CU, each in two K-groups
    (8, 256, 1024, 4096),    # 64 of them, in two K-groups and four K splits
])
def test_gemm_against_oracle(zest_gpu, oracle, wtype, M, N, K):
    import torch
    quant = load_quant()
    x = Rng(M + N).normal(M * K).reshape(M, K)
    w = Rng(M + K).normal(N * K, 0, 0.02).reshape(N, K)
    raw = quant.quantize(wtype, torch.from_numpy(w)).numpy() if wtype else w.view(np.uint8)
    c, nf, a, wp = run_gemm(zest_gpu, x, wtype, raw, N)
    assert nf == 0
    ad = decoded_act(zest_gpu, oracle, a, M, K)
    assert np.array_equal(ad.view(np.uint32), oracle.decode_rows(oracle.encode_rows(x)).view(np.uint32))
    wd = decoded(zest_gpu, oracle, wp, N, K)
    rows = np.arange(M) if M * N * K <= 4e9 else np.linspace(0, M - 1, 96).astype(int)
    r64, ab = oracle.mul_mat_f64(wd, ad[rows])
    worst, maxrel = gemm_check(c[rows], r64, ab, K)
    assert worst <= 1.0, worst
    assert maxrel <= 1e-3, maxrel
    # and against the reference loop itself (xdna-ref's fp32 sequential dot)
    ref32 = oracle.mul_mat_f32(wd, ad[rows[:32]])
    _, maxrel32 = gemm_check(c[rows[:32]], ref32.astype(np.float64), ab[:32], K)
    assert maxrel32 <= 1e-3


def test_gemm_full_size_ffn_properties(zest_gpu, oracle):
    # BASELINE config 2 sizes: gate 2048 x 9728 x 2560 with 1% outlier
    # channels; checked on sampled rows, plus linearity in the activations
    import torch
    quant = load_quant()
    M, N, K = 2048, 9728, 2560
    rng = Rng(21)
    x = rng.normal(M * K).reshape(M, K)
    x[:, rng.ints(K // 100, 0, K - 1)] *= 20.0
    w = Rng(22).normal(N * K, 0, 0.02).reshape(N, K)
    raw = quant.quantize(12, torch.from_numpy(w).cuda()).cpu().numpy()
    c, nf, a, wp = run_gemm(zest_gpu, x, 12, raw, N)
    assert nf == 0
    rows = np.array([0, 1, 2, 511, 1024, 1500, 2046, 2047])
    ad = decoded_act(zest_gpu, oracle, a, M, K)[rows]
    wd = decoded(zest_gpu, oracle, wp, N, K)
    r64, ab = oracle.mul_mat_f64(wd, ad)
    worst, maxrel = gemm_check(c[rows], r64, ab, K)
    assert worst <= 1.0 and maxrel <= 1e-3
    # scaling the activations by 2^j shifts every exponent byte: outputs scale exactly
    c2, _, _, _ = run_gemm(zest_gpu, x * 4.0, 12, raw, N)
    assert np.array_equal(c2, c * 4.0)


def test_nonfinite_flag(zest_gpu):
    import torch
    m, k, n = 64, 128, 256
    x = Rng(1).normal(m * k).reshape(m, k)
    w = Rng(2).normal(n * k).reshape(n, k)
    _, nf, a, wp = run_gemm(zest_gpu, x, 0, w.view(np.uint8), n)
    assert nf == 0
    x[5, 17] = np.inf
    c, nf, _, _ = run_gemm(zest_gpu, x, 0, w.view(np.uint8), n)
    assert nf == 1


def test_gemm_wide_exponent_data(zest_gpu, oracle):
    # make_data's wide exponents 2^-24..2^12 in both operands
    m, k, n = 256, 1024, 512
    x = make_data(m * k, 77).reshape(m, k)
    w = make_data(n * k, 78).reshape(n, k)
    c, nf, a, wp = run_gemm(zest_gpu, x, 0, w.view(np.uint8), n)
    ad = decoded_act(zest_gpu, oracle, a, m, k)
    wd = decoded(zest_gpu, oracle, wp, n, k)
    r64, ab = oracle.mul_mat_f64(wd, ad)
    worst, _ = gemm_check(c, r64, ab, k)
    assert worst <= 1.0


def test_split_k_deterministic_and_reusable(zest_gpu, oracle):
    # launches whose whole tiles would leave CUs idle split K over workgroups;
    # a split tile is summed in split order by whichever workgroup finishes
    # last. The sums must not depend on which one that is, and each launch
    # must leave the per-tile counters at zero for the next: three rounds
    # over three such shapes give the same bits every time.
    import torch
    shapes = [(2048, 2048, 9728), (1024, 2560, 16384), (600, 1000, 8192)]
    runs = {}
    for (M, N, K) in shapes:
        x = Rng(M + 7).normal(M * K).reshape(M, K)
        w = Rng(N + 7).normal(N * K, 0, 0.02).reshape(N, K)
        c, nf, a, wp = run_gemm(zest_gpu, x, 0, w.view(np.uint8), N)
        assert nf == 0
        rows = np.array([0, 1, M // 2, M - 1])
        r64, ab = oracle.mul_mat_f64(decoded(zest_gpu, oracle, wp, N, K), decoded_act(zest_gpu, oracle, a, M, K)[rows])
        worst, maxrel = gemm_check(c[rows], r64, ab, K)
        assert worst <= 1.0 and maxrel <= 1e-3, (M, N, K)
        runs[(M, N, K)] = (a, wp, torch.from_numpy(c))
    for _ in range(2):
        for (M, N, K), (a, wp, c0) in runs.items():
            c = zest_gpu.gemm(a, M, wp, N, K)
            torch.cuda.synchronize()
            assert torch.equal(c.cpu(), c0), (M, N, K)


@pytest.mark.parametrize("M,K,ns,wtype", [
    (2048, 2560, [4096, 1024, 1024], 12),   # config 2's q, k and v
    (300, 200, [200, 96, 1000, 8], 0),      # ragged widths, four weights
    (64, 512, [256], 8),
])
def test_gemm_group(zest_gpu, oracle, M, K, ns, wtype):
    # one launch over weights sharing the activations, against the oracle and
    # against each weight's own launch
    import torch
    quant = load_quant()
    x = Rng(M + K).normal(M * K).reshape(M, K)
    a = zest_gpu.pack_act_x(_dev(x))
    ws, wds = [], []
    for i, n in enumerate(ns):
        w = Rng(100 + i).normal(n * K, 0, 0.02).reshape(n, K)
        raw = quant.quantize(wtype, torch.from_numpy(w)).numpy() if wtype else w.view(np.uint8)
        ws.append(zest_gpu.convert_weight(wtype, _dev(raw), n, K))
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    outs = zest_gpu.gemm_group(a, M, ws, ns, K, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    rows = np.unique(np.linspace(0, M - 1, min(M, 48)).astype(int))
    ad = decoded_act(zest_gpu, oracle, a, M, K)[rows]
    for i, n in enumerate(ns):
        got = outs[i].cpu().numpy()
        r64, ab = oracle.mul_mat_f64(decoded(zest_gpu, oracle, ws[i], n, K), ad)
        worst, maxrel = gemm_check(got[rows], r64, ab, K)
        assert worst <= 1.0 and maxrel <= 1e-3, i
        alone = zest_gpu.gemm(a, M, ws[i], n, K).cpu().numpy()[rows]
        worst, _ = gemm_check(got[rows], alone.astype(np.float64), ab, K)
        assert worst <= 1.0, i


@pytest.mark.parametrize("M,ns,K", [
    (2000, [2560], 4096),         # config 3's O projection with ragged rows: 256 tiles of 128 x 160
    (1024, [5120], 1024),
    (1500, [1600, 1760], 1024),   # a group of two weights, 252 tiles
    (2048, [2560], 9728),         # config 3's down projection: one unsplit round, not three K splits
])
def test_gemm_160_row_tiles(zest_gpu, oracle, M, ns, K):
    # a launch that 256 x 128 tiles run in one round, unsplit, while 128 x 128
    # tiles would take two, runs as 128 x 160 tiles when every weight is whole
    # 160-row tiles: against the oracle; with the residual epilogue (rows past
    # M of the residual holding NaN), bit for bit the GEMM followed by the ADD
    import torch
    x = Rng(M + 7).normal(M * K).reshape(M, K)
    a = zest_gpu.pack_act_x(_dev(x))
    ws = []
    for i, n in enumerate(ns):
        w = Rng(n + 7 + i).normal(n * K, 0, 0.02).reshape(n, K)
        ws.append(zest_gpu.convert_weight(0, _dev(w.view(np.uint8)), n, K))
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    outs = zest_gpu.gemm_group(a, M, ws, ns, K, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    rows = np.unique(np.concatenate([np.linspace(0, M - 1, 40).astype(int), [127, 128, M - 1]]))
    ad = decoded_act(zest_gpu, oracle, a, M, K)[rows]
    for i, n in enumerate(ns):
        r64, ab = oracle.mul_mat_f64(decoded(zest_gpu, oracle, ws[i], n, K), ad)
        worst, maxrel = gemm_check(outs[i].cpu().numpy()[rows], r64, ab, K)
        assert worst <= 1.0 and maxrel <= 1e-3, i
    if len(ns) == 1:
        N = ns[0]
        big = torch.full((M + 64, N), float("nan"), device="cuda")
        big[:M] = torch.from_numpy(Rng(M * 5).normal(M * N).reshape(M, N)).cuda()
        want = zest_gpu.add(outs[0], big[:M].contiguous())
        got = zest_gpu.gemm_residual(a, M, ws[0], N, K, big[:M], nonfinite=nf)
        torch.cuda.synchronize()
        assert int(nf.item()) == 0
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("M,ns,K", [
    (4000, [2048, 1024, 1024], 512),  # 16 x 32 = 512 tiles of 256 x 128: two rounds, persistent workgroups
    (2048, [4096, 4096, 4096], 1024),  # 8 x 96 = 768 tiles: three rounds
    (4000, [2048, 1024, 1024], 576),  # an odd number of K-steps: one workgroup a tile
    (4096, [4096, 1024], 512),  # 640 tiles: two rounds and a half, the half as 128-row tiles (each workgroup two whole, one half)
])
def test_gemm_rounds_equal_one_round_launches(zest_gpu, oracle, M, ns, K):
    # A launch of more than one round of whole tiles, unsplit, runs as
    # persistent workgroups that take their XCD's tiles in turn and fetch the
    # next tile's first steps during the current one. Every output is summed
    # over K in the same order as in a launch of one round, so the group
    # launch equals, bit for bit, each weight launched alone (at most one
    # round), and it meets the oracle's bar. The operands' blocks spread over
    # 2^+-12, so a change of summation order would show.
    import torch
    x = wide_blocks(M, K, M + K)
    a = zest_gpu.pack_act_x(_dev(x))
    ws = [zest_gpu.convert_weight(0, _dev(wide_blocks(n, K, n + i + K, 0.02).view(np.uint8)), n, K)
          for i, n in enumerate(ns)]
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    outs = zest_gpu.gemm_group(a, M, ws, ns, K, nonfinite=nf)
    alone = [zest_gpu.gemm(a, M, w, n, K) for w, n in zip(ws, ns)]
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    for i in range(len(ns)):
        assert torch.equal(outs[i].view(torch.int32), alone[i].view(torch.int32)), i
    rows = np.unique(np.concatenate([np.linspace(0, M - 1, 32).astype(int), [255, 256, M - 1]]))
    ad = decoded_act(zest_gpu, oracle, a, M, K)[rows]
    r64, ab = oracle.mul_mat_f64(decoded(zest_gpu, oracle, ws[-1], ns[-1], K), ad)
    worst, _ = gemm_check(outs[-1].cpu().numpy()[rows], r64, ab, K)
    assert worst <= 1.0


def test_gemm_part_round_as_half_tiles(zest_gpu, oracle):
    # M = 2048, N = 6144: 384 tiles of 256 x 128, one round of the GPU's 256
    # CUs and half of another; the launch runs the last 128 tiles as 256 of
    # 128 x 128. Each output is summed over K in the same order either way, so
    # the result equals, bit for bit, two launches over the column halves (192
    # whole tiles each), and the oracle within the GEMM bar. Order-sensitive
    # operands (blocks spread over 2^+-12).
    M, N, K = 2048, 6144, 512
    x = wide_blocks(M, K, 3)
    w = wide_blocks(N, K, 4, 0.02)
    c, nf, a, wp = run_gemm(zest_gpu, x, 0, w.view(np.uint8), N)
    assert nf == 0
    half = N // 2
    parts = [zest_gpu.gemm(a, M, zest_gpu.convert_weight(0, _dev(np.ascontiguousarray(w[h * half:(h + 1) * half])
                                                                 .view(np.uint8)), half, K), half, K)
             for h in range(2)]
    both = np.concatenate([q.cpu().numpy() for q in parts], axis=1)
    assert np.array_equal(c.view(np.uint32), both.view(np.uint32))
    rows = np.unique(np.concatenate([np.linspace(0, M - 1, 40).astype(int), [1024, 1151, 1152, 1279, 2047]]))
    r64, ab = oracle.mul_mat_f64(decoded(zest_gpu, oracle, wp, N, K), decoded_act(zest_gpu, oracle, a, M, K)[rows])
    worst, _ = gemm_check(c[rows], r64, ab, K)
    assert worst <= 1.0


def test_gemm_group_rejects_bad_counts(zest_gpu):
    import torch
    a = zest_gpu.empty_act(64, 64)
    w = zest_gpu.empty_packed(128, 64)
    with pytest.raises(RuntimeError):
        zest_gpu.gemm_group(a, 64, [w] * 5, [128] * 5, 64)
    with pytest.raises(RuntimeError):
        zest_gpu.gemm_group(a, 64, [], [], 64)
    torch.cuda.synchronize()


@pytest.mark.parametrize("M,N,K", [
    (2048, 2560, 4096),   # config 3's O projection: h += O
    (2048, 2560, 9728),   # its down projection (one round of 128 x 160 tiles)
    (300, 200, 256),      # ragged rows, 128x128 tiles
    (1024, 1000, 512),    # a width that is not a tile multiple
    (2048, 6144, 512),    # 384 tiles: a round and a half, the half as 128-row tiles
    (1024, 1024, 4096),   # 64x64 tiles in two K-groups
    (256, 1024, 4096),    # and in four K splits
])
def test_gemm_residual_is_gemm_then_add(zest_gpu, M, N, K):
    # the residual epilogue adds in the store: the same floats as the GEMM
    # followed by the ADD kernel, in place (res is the output) or not
    import torch
    x = Rng(M + 11).normal(M * K).reshape(M, K)
    w = Rng(N + 11).normal(N * K, 0, 0.02).reshape(N, K)
    a = zest_gpu.pack_act_x(_dev(x))
    wp = zest_gpu.convert_weight(0, _dev(w.view(np.uint8)), N, K)
    h0 = torch.from_numpy(Rng(M + N).normal(M * N).reshape(M, N)).cuda()
    want = zest_gpu.add(zest_gpu.gemm(a, M, wp, N, K), h0)
    out = zest_gpu.gemm_residual(a, M, wp, N, K, h0)
    h = h0.clone()
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    zest_gpu.gemm_residual(a, M, wp, N, K, h, out=h, nonfinite=nf)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), want.view(torch.int32))
    assert torch.equal(h.view(torch.int32), want.view(torch.int32))
    assert int(nf.item()) == 0


@pytest.mark.parametrize("M,N,K", [(300, 200, 256), (1000, 2560, 4096), (2047, 2560, 9728)])
def test_residual_ragged_rows_ignore_what_follows(zest_gpu, M, N, K):
    # the residual is the first M rows of a larger buffer whose other rows
    # hold NaN (as memory after a tensor may): the epilogue's reads of rows
    # past M must come back as zeros and stay out of the non-finite flag, and
    # the rows past M must not be written
    import torch
    x = Rng(M + 5).normal(M * K).reshape(M, K)
    w = Rng(N + 5).normal(N * K, 0, 0.02).reshape(N, K)
    a = zest_gpu.pack_act_x(_dev(x))
    wp = zest_gpu.convert_weight(0, _dev(w.view(np.uint8)), N, K)
    big = torch.full((M + 64, N), float("nan"), device="cuda")
    big[:M] = torch.from_numpy(Rng(M * 3).normal(M * N).reshape(M, N)).cuda()
    res = big[:M]
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    want = zest_gpu.add(zest_gpu.gemm(a, M, wp, N, K), res.contiguous())
    outbig = torch.full((M + 64, N), float("nan"), device="cuda")
    zest_gpu.gemm_residual(a, M, wp, N, K, res, out=outbig[:M], nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    assert torch.equal(outbig[:M].view(torch.int32), want.view(torch.int32))
    assert bool(torch.isnan(outbig[M:]).all())


def test_gemm_random_shapes(zest_gpu, oracle):
    # a seeded sweep over odd shapes (rows from 1 to a few rounds of tiles,
    # widths in steps of 32, K in steps of 8) through the plain, residual and
    # grouped launches, against the oracle within the GEMM bar, and the fused
    # GLU bit-exact with the unfused chain over the same GEMM; the launch picks
    # tile shapes, splits and mixed rounds as it would for any caller
    import torch
    rng = np.random.default_rng(20260)
    for case in range(24):
        M = int(rng.choice([1, 7, 100, 129, 300, 513, 1000, 1500, 2100]))
        N = int(rng.integers(1, 64)) * 32 * int(rng.choice([1, 2, 4]))
        K = int(rng.integers(1, 40)) * 8 * int(rng.choice([1, 2, 4]))
        x = rng.normal(0, 1, (M, K)).astype(np.float32)
        w = rng.normal(0, 0.05, (N, K)).astype(np.float32)
        a = zest_gpu.pack_act_x(_dev(x))
        kind = case % 4
        if kind == 3:
            # order-sensitive operands: blocks spread over 2^+-12
            F = max(32, N // 64 * 32)
            x = wide_blocks(M, K, 1000 + case)
            a = zest_gpu.pack_act_x(_dev(x))
            gate, up = wide_blocks(F, K, 2000 + case, 0.05), wide_blocks(F, K, 3000 + case, 0.05)
            wgu = zest_gpu.convert_weight_gu(0, _dev(gate.view(np.uint8)), _dev(up.view(np.uint8)), F, K)
            c = zest_gpu.gemm(a, M, wgu, 2 * F, K).view(M, F // 32, 2, 32)
            h_ref = zest_gpu.glu(2, c[:, :, 0, :].reshape(M, F).contiguous(), c[:, :, 1, :].reshape(M, F).contiguous(), F)
            nf = torch.zeros(1, dtype=torch.int32, device="cuda")
            xo, h = zest_gpu.gemm_glu(2, a, M, wgu, F, K, h=True, nonfinite=nf)
            x_ref = zest_gpu.pack_act_x(h_ref)
            torch.cuda.synchronize()
            assert int(nf.item()) == 0, (M, F, K)
            assert torch.equal(h.view(torch.int32), h_ref.view(torch.int32)), (M, F, K)
            assert torch.equal(xo, x_ref), (M, F, K)
            continue
        wp = zest_gpu.convert_weight(0, _dev(w.view(np.uint8)), N, K)
        slack = 0.0
        if kind == 0:
            got = zest_gpu.gemm(a, M, wp, N, K).cpu().numpy().astype(np.float64)
        elif kind == 1:
            res = rng.normal(0, 1, (M, N)).astype(np.float32)
            nf = torch.zeros(1, dtype=torch.int32, device="cuda")
            out = zest_gpu.gemm_residual(a, M, wp, N, K, _dev(res), nonfinite=nf).cpu().numpy().astype(np.float64)
            assert int(nf.item()) == 0, (M, N, K)
            got, slack = out - res, np.abs(out) * 2.0 ** -24  # the add rounds once more
        else:
            cuts = sorted({0, N, *(int(v) // 8 * 8 for v in rng.integers(8, max(9, N - 8), 2))})
            parts = [(lo, hi) for lo, hi in zip(cuts, cuts[1:]) if hi > lo]
            ws = [zest_gpu.convert_weight(0, _dev(np.ascontiguousarray(w[lo:hi]).view(np.uint8)), hi - lo, K)
                  for lo, hi in parts]
            outs = zest_gpu.gemm_group(a, M, ws, [hi - lo for lo, hi in parts], K)
            got = np.concatenate([o.cpu().numpy() for o in outs], axis=1).astype(np.float64)
        rows = np.unique(np.linspace(0, M - 1, min(M, 16)).astype(int))
        r64, ab = oracle.mul_mat_f64(decoded(zest_gpu, oracle, wp, N, K), decoded_act(zest_gpu, oracle, a, M, K)[rows])
        sl = slack[rows] if kind == 1 else 0.0
        err = np.abs(got[rows] - r64)
        bound = 2.0 * K * 2.0 ** -24 * ab + sl
        assert np.isfinite(got[rows]).all() and (err <= bound).all(), (kind, M, N, K, float((err / bound).max()))



def test_gemm_random_shapes_order_sensitive(zest_gpu, oracle):
    # a wider seeded sweep on operands whose 8-value blocks span 2^+-12: rows
    # up to a few rounds of tiles (and across the 64-, 256- and 1024-row
    # boundaries), widths up to 12288, K up to 4096, so the planner takes
    # every tile shape, K split and K-group form; the plain, grouped and
    # residual launches against the oracle's bound, the residual added in
    # place bit-exact with the GEMM then ADD, and the fused GLU of every kind
    # bit-exact with the unfused chain, its operand written whole (padding
    # included) into a buffer that held garbage
    import torch
    z = zest_gpu
    rng = np.random.default_rng(31337)
    for case in range(48):
        M = int(rng.choice([1, 5, 64, 65, 200, 256, 257, 511, 768, 1024, 1025, 1536, 2048, 3000, 4096]))
        N = int(rng.integers(1, 96)) * 32 * int(rng.choice([1, 2, 4]))
        K = int(rng.integers(1, 64)) * 8 * int(rng.choice([1, 2, 4, 8]))
        kind = case % 5
        x = wide_blocks(M, K, 10_000 + case)
        a = z.pack_act_x(_dev(x))
        if kind == 4:
            F = max(32, N // 64 * 32)
            gate, up = wide_blocks(F, K, 20_000 + case, 0.05), wide_blocks(F, K, 30_000 + case, 0.05)
            wgu = z.convert_weight_gu(0, _dev(gate.view(np.uint8)), _dev(up.view(np.uint8)), F, K)
            c = z.gemm(a, M, wgu, 2 * F, K).view(M, F // 32, 2, 32)
            gk = int(rng.integers(0, 5))
            h_ref = z.glu(gk, c[:, :, 0, :].reshape(M, F).contiguous(), c[:, :, 1, :].reshape(M, F).contiguous(), F)
            x_ref = z.pack_act_x(h_ref)
            buf = torch.full_like(x_ref, 0xFF)
            xo, h = z.gemm_glu(gk, a, M, wgu, F, K, xout=buf, h=True)
            torch.cuda.synchronize()
            assert torch.equal(h.view(torch.int32), h_ref.view(torch.int32)), (gk, M, F, K)
            assert torch.equal(buf, x_ref), (gk, M, F, K)
            continue
        w = wide_blocks(N, K, 40_000 + case, 0.05)
        wp = z.convert_weight(0, _dev(w.view(np.uint8)), N, K)
        res = rng.normal(0, 1, (M, N)).astype(np.float32)
        if kind == 3:
            want = z.add(z.gemm(a, M, wp, N, K), _dev(res))
            h0 = _dev(res)
            z.gemm_residual(a, M, wp, N, K, h0, out=h0)
            torch.cuda.synchronize()
            assert torch.equal(h0.view(torch.int32), want.view(torch.int32)), (M, N, K)
            continue
        slack = 0.0
        if kind == 0:
            got = z.gemm(a, M, wp, N, K).cpu().numpy().astype(np.float64)
        elif kind == 1:
            out = z.gemm_residual(a, M, wp, N, K, _dev(res)).cpu().numpy().astype(np.float64)
            got, slack = out - res, np.abs(out) * 2.0 ** -24  # the add rounds once more
        else:
            cuts = sorted({0, N, *(int(v) // 8 * 8 for v in rng.integers(8, max(9, N - 8), 2))})
            parts = [(lo, hi) for lo, hi in zip(cuts, cuts[1:]) if hi > lo]
            ws = [z.convert_weight(0, _dev(np.ascontiguousarray(w[lo:hi]).view(np.uint8)), hi - lo, K)
                  for lo, hi in parts]
            outs = z.gemm_group(a, M, ws, [hi - lo for lo, hi in parts], K)
            got = np.concatenate([o.cpu().numpy() for o in outs], axis=1).astype(np.float64)
        rows = np.unique(np.linspace(0, M - 1, min(M, 12)).astype(int))
        r64, ab = oracle.mul_mat_f64(decoded(z, oracle, wp, N, K), decoded_act(z, oracle, a, M, K)[rows])
        sl = slack[rows] if kind == 1 else 0.0
        err = np.abs(got[rows] - r64)
        bound = 2.0 * K * 2.0 ** -24 * ab + sl
        assert np.isfinite(got[rows]).all() and (err <= bound).all(), (kind, M, N, K, float((err / bound).max()))


def test_gemm_output_bands(zest_gpu, oracle):
    # an output whose span passes 2 GiB (the all-logits projection: vocab
    # 151,936 at a 4096-token ubatch, 2.49 GB of fp32) runs as launches over
    # bands of 3328 rows (13 tiles of 256 rows under 2 GiB each); rows on both
    # sides of the band edge and the ragged end are checked against the
    # oracle, the residual epilogue's bands bit for bit against the plain
    # bands plus the add, and a group launch with a narrow weight beside the
    # wide one against the oracle
    import torch
    quant = load_quant()
    M, N, K = 4096, 151936, 512
    assert M * N * 4 >= 2 ** 31
    x = Rng(151).normal(M * K).reshape(M, K)
    w = Rng(152).normal(N * K, 0, 0.02).reshape(N, K)
    raw = quant.quantize(8, torch.from_numpy(w).cuda())
    a = zest_gpu.pack_act_x(_dev(x))
    wp = zest_gpu.convert_weight(8, raw, N, K)
    del raw
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    c = zest_gpu.gemm(a, M, wp, N, K, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    rows = np.array([0, 1, 1000, 3326, 3327, 3328, 3329, 3583, 3584, 4094, 4095])
    got = c[torch.from_numpy(rows).cuda()].cpu().numpy()
    ad = decoded_act(zest_gpu, oracle, a, M, K)[rows]
    wd = decoded(zest_gpu, oracle, wp, N, K)
    r64, ab = oracle.mul_mat_f64(wd, ad)
    del wd
    worst, maxrel = gemm_check(got, r64, ab, K)
    assert worst <= 1.0, worst
    assert maxrel <= 1e-3, maxrel
    # the residual epilogue over the same bands: acc + res, added once
    res = torch.empty_like(c).normal_()
    out = zest_gpu.gemm_residual(a, M, wp, N, K, res, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    sel = torch.from_numpy(rows).cuda()
    assert torch.equal(out[sel].view(torch.int32), (c[sel] + res[sel]).view(torch.int32))
    del out, res
    # a group: the wide weight beside a narrow one, banded on the widest row
    wn = zest_gpu.convert_weight(8, quant.quantize(8, torch.from_numpy(w[:512]).cuda()), 512, K)
    outs = zest_gpu.gemm_group(a, M, [wn, wp], [512, N], K)
    torch.cuda.synchronize()
    assert gemm_check(outs[1][sel].cpu().numpy(), r64, ab, K)[0] <= 1.0
    n64, nab = oracle.mul_mat_f64(oracle.decode_rows(zest_gpu.tiles_to_blocks(wn.cpu().numpy(), 512, K)), ad)
    assert gemm_check(outs[0][sel].cpu().numpy(), n64, nab, K)[0] <= 1.0


def test_release_stream_frees_and_regrows_the_split_k_workspace(zest_gpu, oracle):
    # a few tiles over a long K: the plan splits K among workgroups, which
    # takes the stream's workspace; released, the next call on the stream
    # allocates it again and computes the same bits
    import torch
    M, N, K = 64, 512, 16384
    x = wide_blocks(M, K, 5)
    w = wide_blocks(N, K, 6, 0.02)
    a = zest_gpu.pack_act_x(_dev(x))
    wp = zest_gpu.convert_weight(0, _dev(w.view(np.uint8)), N, K)
    lib = zest_gpu.lib()
    s = torch.cuda.Stream()
    outs = []
    with torch.cuda.stream(s):
        for _ in range(2):
            outs.append(zest_gpu.gemm(a, M, wp, N, K))
            assert lib.zest_release_stream(s.cuda_stream) == 0
            assert lib.zest_release_stream(s.cuda_stream) == 0      # nothing held any more
    s.synchronize()
    assert lib.zest_release_stream(None) == 0                       # the null stream's, if any
    c0, c1 = (o.cpu().numpy() for o in outs)
    assert np.array_equal(c0.view(np.uint32), c1.view(np.uint32))
    rows = np.arange(0, M, 7)
    r64, ab = oracle.mul_mat_f64(decoded(zest_gpu, oracle, wp, N, K), decoded_act(zest_gpu, oracle, a, M, K)[rows])
    worst, _ = gemm_check(c0[rows], r64, ab, K)
    assert worst <= 1.0
