"""The fused gate/up GEMM (zest_convert_weight_gu + zest_gemm_glu): the
reference's fused SwiGLU matmul (src/xdna-exec.cpp:399-431, output mode 2 of
kernels/bfp16_gemm/aie_kernels/aie2p/mm_bfp_acc.cc:258-278).

Its result must be bit-exact with the unfused chain over the same GEMM:
zest_gemm of the interleaved weight (pinned against the oracle in
test_gemm_gpu), whose gate and up columns go through zest_glu (pinned in
test_ops_gpu) and zest_pack_act_x (bit-exact with the oracle's encoder in
test_pack_gpu). The fused launch splits K among workgroups, and among the
K-groups of a workgroup, exactly as the plain launch of its 2F columns does
(whatever tile shapes the two take), so each output is summed over K in the
same order and every float matches. The
bit-exact tests that could miss a change of summation order use operands
whose 8-value blocks span 2^+-12 (fp32 partial sums of their products are
rarely exact), and a control shows that with them another K partition does
change bits. Against
the chain the reference runs unfused (separate gate and up GEMMs, whose
launches can split K differently) and against the oracle, h must meet the
host ops' bar (nrmse <= 1e-5, tests/test-host-ops.cpp).
"""
from __future__ import annotations

import numpy as np
import pytest
from gen import Rng, wide_blocks
from helpers import load_quant, nrmse

pytestmark = pytest.mark.gpu

KINDS = {"reglu": 0, "geglu": 1, "swiglu": 2, "geglu_erf": 3, "geglu_quick": 4}


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _weights(wtype: int, f: int, k: int, seed: int):
    """Gate and up GGUF rows (uint8 device tensors) of `wtype`."""
    import torch
    quant = load_quant()
    out = []
    for s in (seed, seed + 1):
        w = Rng(s).normal(f * k, 0, 0.05).reshape(f, k)
        raw = quant.quantize(wtype, torch.from_numpy(w).cuda()).cpu().numpy() if wtype else w.view(np.uint8)
        out.append(_dev(raw))
    return out


def unfused(z, kind, a, m, wgu, f, k):
    """The plain GEMM over the interleaved weight, its gate and up columns
    through the GLU kernel, then the down projection's operand."""
    c = z.gemm(a, m, wgu, 2 * f, k).view(m, f // 32, 2, 32)
    g = c[:, :, 0, :].reshape(m, f).contiguous()
    u = c[:, :, 1, :].reshape(m, f).contiguous()
    h = z.glu(kind, g, u, f)
    return z.pack_act_x(h), h, g, u


def separate(z, kind, a, m, gate, up, wtype, f, k):
    """The chain without any fusion: two weights, two GEMMs, the GLU."""
    g = z.gemm(a, m, z.convert_weight(wtype, gate, f, k), f, k)
    u = z.gemm(a, m, z.convert_weight(wtype, up, f, k), f, k)
    return z.glu(kind, g, u, f)


@pytest.mark.parametrize("wtype,M,F,K", [
    (0, 300, 96, 200),      # F % 64 == 32: half a K-tile of the output operand is padding
    (0, 37, 64, 64),
    (8, 1024, 2560, 1536),
    (12, 520, 8960 // 10, 1536),
    (12, 2048, 9728, 2560),  # BASELINE config 2's gate/up: 2048 x 9728 x 2560, Q4_K
    (8, 2048, 1024, 9728),   # few tiles, long K: the launch splits K
    (0, 2048, 3072, 512),    # 384 tiles: a round and a half, the half as 128-row tiles
    (0, 1500, 4096, 512),    # 6 x 64 = 384 tiles, ragged rows: persistent workgroups
])
def test_gemm_glu_matches_unfused_swiglu(zest_gpu, oracle, wtype, M, F, K):
    import torch
    x = Rng(M + F + K).normal(M * K).reshape(M, K)
    gate, up = _weights(wtype, F, K, F + K)
    a = zest_gpu.pack_act_x(_dev(x))
    wgu = zest_gpu.convert_weight_gu(wtype, gate, up, F, K)
    x_ref, h_ref, g, u = unfused(zest_gpu, 2, a, M, wgu, F, K)
    h_sep = separate(zest_gpu, 2, a, M, gate, up, wtype, F, K)
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    xo, h = zest_gpu.gemm_glu(2, a, M, wgu, F, K, h=True, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    assert torch.equal(h.view(torch.int32), h_ref.view(torch.int32))
    assert torch.equal(xo, x_ref)
    assert nrmse(h.cpu().numpy(), h_sep.cpu().numpy()) <= 1e-5
    # the operand's values are the oracle's bfp16 encoding of h (sampled rows)
    rows = np.unique(np.linspace(0, M - 1, min(M, 64)).astype(int))
    hs = h.cpu().numpy()[rows]
    xd = zest_gpu.expanded_to_rows(xo.cpu().numpy(), M, F)[rows]
    assert np.array_equal(xd.view(np.uint32), oracle.decode_rows(oracle.encode_rows(hs)).view(np.uint32))
    # and h is the oracle's SwiGLU of the gate and up products
    gs, us = g.cpu().numpy()[rows], u.cpu().numpy()[rows]
    assert nrmse(hs, oracle.glu(2, gs, us)) <= 1e-5  # tests/test-host-ops.cpp's bar


def _wide_case(z, M, F, K, seed):
    """Order-sensitive operands: activations and F32 gate/up weights with
    8-value blocks spread over 2^+-12."""
    x = wide_blocks(M, K, seed)
    gate = _dev(wide_blocks(F, K, seed + 1, 0.05).view(np.uint8))
    up = _dev(wide_blocks(F, K, seed + 2, 0.05).view(np.uint8))
    a = z.pack_act_x(_dev(x))
    return a, z.convert_weight_gu(0, gate, up, F, K)


def test_order_sensitive_operands_show_another_k_split(zest_gpu):
    # The control for the bit-exact tests below: with these operands the same
    # GEMM summed over another partition of K (two launches over the halves
    # of K, added in fp32) differs from the one-launch sums in many outputs,
    # so a fused launch that split K otherwise than the plain one would fail
    # its bit-exact test. (With N(0,1) activations and small weights, every
    # fp32 partial sum is exact and no order change would show.)
    import torch
    M, N, K = 512, 512, 4096
    x = wide_blocks(M, K, 61)
    w = wide_blocks(N, K, 62, 0.05)
    a = zest_gpu.pack_act_x(_dev(x))
    full = zest_gpu.gemm(a, M, zest_gpu.convert_weight(0, _dev(w.view(np.uint8)), N, K), N, K)
    h = K // 2
    halves = None
    for lo in (0, h):
        ah = zest_gpu.pack_act_x(_dev(np.ascontiguousarray(x[:, lo:lo + h])))
        wh = zest_gpu.convert_weight(0, _dev(np.ascontiguousarray(w[:, lo:lo + h]).view(np.uint8)), N, h)
        part = zest_gpu.gemm(ah, M, wh, N, h)
        halves = part if halves is None else halves + part
    torch.cuda.synchronize()
    differ = float((full.view(torch.int32) != halves.view(torch.int32)).float().mean())
    assert differ > 0.1, differ
    assert torch.allclose(full, halves, rtol=1e-4, atol=float(full.abs().max()) * 1e-5)


@pytest.mark.parametrize("M,F,K", [
    (520, 896, 1536),   # 252 tiles of 64x64, each K-split between two K-groups
    (1024, 512, 4096),  # 256 of them, K 4096
    (2048, 1024, 8192),  # few tiles, long K: split
    (256, 512, 4096),    # 64 tiles of 64x64 in two K-groups and four K splits
    (2048, 6144, 4096),  # three rounds: persistent workgroups
    (1500, 4096, 4096),
])
def test_gemm_glu_bit_exact_order_sensitive(zest_gpu, M, F, K):
    # the fused gate/up sums are the plain GEMM's over the interleaved weight
    # bit for bit, on operands where a change of K summation order shows
    import torch
    a, wgu = _wide_case(zest_gpu, M, F, K, M + F + K)
    x_ref, h_ref, _, _ = unfused(zest_gpu, 2, a, M, wgu, F, K)
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    xo, h = zest_gpu.gemm_glu(2, a, M, wgu, F, K, h=True, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    assert torch.equal(h.view(torch.int32), h_ref.view(torch.int32)), (M, F, K)
    assert torch.equal(xo, x_ref), (M, F, K)


@pytest.mark.parametrize("M,F,K", [
    (65, 96, 2560),     # 64x64 tiles in K-groups and K splits; F % 64 == 32
    (300, 96, 200),     # 128-column tiles; F % 64 == 32
    (1024, 160, 4096),  # 64x64 tiles in K-groups; F % 64 == 32
])
def test_gemm_glu_writes_the_operand_padding(zest_gpu, M, F, K):
    # the fused launch writes every byte of the down projection's operand,
    # the K padding past F (half a 64-column K-tile here) and the rows past
    # M included, into a buffer that held garbage: the bytes of
    # zest_pack_act_x over the unfused chain's h
    import torch
    a, wgu = _wide_case(zest_gpu, M, F, K, 7 * M + F)
    x_ref, h_ref, _, _ = unfused(zest_gpu, 2, a, M, wgu, F, K)
    buf = torch.full_like(x_ref, 0xFF)
    xo, _ = zest_gpu.gemm_glu(2, a, M, wgu, F, K, xout=buf)
    torch.cuda.synchronize()
    assert xo.data_ptr() == buf.data_ptr()
    assert torch.equal(buf, x_ref), (M, F, K, int((buf != x_ref).sum()))


@pytest.mark.parametrize("M,F,K", [
    (300, 160, 256),    # 6 tiles: one workgroup a tile
    (1500, 4096, 512),  # 384 tiles: persistent workgroups, each kind's own kernel
])
@pytest.mark.parametrize("kind", list(KINDS))
def test_gemm_glu_every_kind(zest_gpu, kind, M, F, K):
    import torch
    x = Rng(5 + M).normal(M * K).reshape(M, K)
    gate, up = _weights(0, F, K, 9)
    a = zest_gpu.pack_act_x(_dev(x))
    wgu = zest_gpu.convert_weight_gu(0, gate, up, F, K)
    x_ref, h_ref, _, _ = unfused(zest_gpu, KINDS[kind], a, M, wgu, F, K)
    xo, h = zest_gpu.gemm_glu(KINDS[kind], a, M, wgu, F, K, h=True)
    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int32), h_ref.view(torch.int32)), kind
    assert torch.equal(xo, x_ref), kind


def test_gemm_glu_outputs_alone_and_strided(zest_gpu):
    # xout only, h only into rows of a wider buffer: the same values
    import torch
    M, F, K = 700, 320, 512
    x = Rng(11).normal(M * K).reshape(M, K)
    gate, up = _weights(8, F, K, 13)
    a = zest_gpu.pack_act_x(_dev(x))
    wgu = zest_gpu.convert_weight_gu(8, gate, up, F, K)
    xo, h = zest_gpu.gemm_glu(2, a, M, wgu, F, K, h=True)
    xo_only, none = zest_gpu.gemm_glu(2, a, M, wgu, F, K)
    wide = torch.full((M, F + 40), 7.0, device="cuda")
    _, h2 = zest_gpu.gemm_glu(2, a, M, wgu, F, K, xout=None, h=wide)
    torch.cuda.synchronize()
    assert none is None
    assert torch.equal(xo_only, xo)
    assert torch.equal(wide[:, :F], h) and bool((wide[:, F:] == 7.0).all())


def test_gemm_glu_one_weight_gate_then_up(zest_gpu):
    # a GLU over one matmul whose weight holds the gate rows, then the up rows
    # (the reference's Phi case, src/xdna-exec.cpp:402-403)
    import torch
    quant = load_quant()
    M, F, K = 512, 256, 1024
    w = Rng(17).normal(2 * F * K, 0, 0.05).reshape(2 * F, K)
    raw = _dev(quant.quantize(12, torch.from_numpy(w).cuda()).cpu().numpy()).reshape(-1)
    rb = zest_gpu.raw_row_bytes(12, K)
    x = Rng(19).normal(M * K).reshape(M, K)
    a = zest_gpu.pack_act_x(_dev(x))
    wfull = zest_gpu.convert_weight(12, raw, 2 * F, K)
    gu = zest_gpu.gemm(a, M, wfull, 2 * F, K)
    h_sep = zest_gpu.glu(2, gu[:, :F], gu[:, F:], F)
    wgu = zest_gpu.convert_weight_gu(12, raw[:F * rb], raw[F * rb:], F, K)
    x_ref, h_ref, _, _ = unfused(zest_gpu, 2, a, M, wgu, F, K)
    xo, h = zest_gpu.gemm_glu(2, a, M, wgu, F, K, h=True)
    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int32), h_ref.view(torch.int32))
    assert torch.equal(xo, x_ref)
    assert nrmse(h.cpu().numpy(), h_sep.cpu().numpy()) <= 1e-5


def test_convert_weight_gu_is_the_interleaved_pair(zest_gpu):
    # rows 64g..64g+31 of the pair are gate rows 32g.., rows 64g+32.. the up
    # rows: each row's blocks are convert_weight's, and the padding is zero
    for wtype, F, K in [(0, 96, 200), (8, 320, 512), (12, 224, 256)]:
        gate, up = _weights(wtype, F, K, 23)
        pair = zest_gpu.convert_weight_gu(wtype, gate, up, F, K).cpu().numpy()
        bg = zest_gpu.tiles_to_blocks(zest_gpu.convert_weight(wtype, gate, F, K).cpu().numpy(), F, K)
        bu = zest_gpu.tiles_to_blocks(zest_gpu.convert_weight(wtype, up, F, K).cpu().numpy(), F, K)
        rows_pad = zest_gpu.rows_pad(2 * F)
        bp = zest_gpu.tiles_to_blocks(pair, rows_pad, K)
        r = np.arange(F)
        dst = (r // 32) * 64 + r % 32
        assert np.array_equal(bp[dst], bg), wtype
        assert np.array_equal(bp[dst + 32], bu), wtype
        rest = np.setdiff1d(np.arange(rows_pad), np.concatenate([dst, dst + 32]))
        assert not bp[rest].any(), wtype


def test_gemm_glu_nonfinite_flag(zest_gpu):
    import torch
    M, F, K = 64, 64, 128
    x = Rng(29).normal(M * K).reshape(M, K)
    x[3, 5] = np.inf
    gate, up = _weights(0, F, K, 31)
    a = zest_gpu.pack_act_x(_dev(x))
    wgu = zest_gpu.convert_weight_gu(0, gate, up, F, K)
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    zest_gpu.gemm_glu(2, a, M, wgu, F, K, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 1


def test_gemm_glu_rejects_bad_sizes(zest_gpu):
    import torch
    a = zest_gpu.empty_act(64, 64)
    w = zest_gpu.empty_packed(128, 64)
    with pytest.raises(RuntimeError):
        zest_gpu.gemm_glu(2, a, 64, w, 48, 64)          # F % 32 != 0
    with pytest.raises(RuntimeError):
        zest_gpu.gemm_glu(9, a, 64, w, 64, 64)          # no such GLU kind
    with pytest.raises(RuntimeError):
        zest_gpu.gemm_glu(2, a, 64, w, 64, 64, xout=None)  # no output
    torch.cuda.synchronize()
