"""The host-op kernels against the oracle, at the bar of tests/test-host-ops.cpp
(nrmse <= 1e-5 against the CPU's result; inputs N(0, 1.5), rope factors
U(1, 4), positions 5000 + 300 i). The fused packs must be bit-exact with the
reference encoder applied to the kernel's own fp32 result."""
from __future__ import annotations

import numpy as np
import pytest
from gen import Rng
from helpers import nrmse

pytestmark = pytest.mark.gpu

EXACT = 1e-5


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("rows,d", [(8, 256), (2048, 2560), (5, 200), (3, 5120), (40, 6144), (6, 7000), (3, 9728)])
def test_rms_norm_mul_and_fused_pack(zest_gpu, oracle, rows, d):
    import torch
    x = Rng(rows + d).normal(rows * d, 0, 1.5).reshape(rows, d)
    w = Rng(d).normal(d, 1.0, 0.1)
    want = oracle.mul_row(oracle.rms_norm(x, 1e-6), w)
    packed = zest_gpu.empty_act(rows, d)
    y = zest_gpu.rms_norm(_dev(x), 1e-6, _dev(w), packed=packed)
    got = _host(y)
    assert nrmse(got, want) <= EXACT
    if d % 8 == 0:
        # the fused pack: the bfp16 encoding of the normed rows, stored expanded
        pk = zest_gpu.expanded_to_rows(_host(packed), rows, d)
        assert np.array_equal(pk.view(np.uint32), oracle.decode_rows(oracle.encode_rows(got)).view(np.uint32))
    # without the scale row: plain RMS_NORM
    y2 = zest_gpu.rms_norm(_dev(x), 1e-6)
    assert nrmse(_host(y2), oracle.rms_norm(x, 1e-6)) <= EXACT
    del torch


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4])
def test_glu_split(zest_gpu, oracle, kind):
    rows, f = 8, 256
    g = Rng(50 + kind).normal(rows * f, 0, 1.5).reshape(rows, f)
    u = Rng(60 + kind).normal(rows * f, 0, 1.5).reshape(rows, f)
    got = _host(zest_gpu.glu(kind, _dev(g), _dev(u), f))
    assert nrmse(got, oracle.glu(kind, g, u)) <= EXACT


@pytest.mark.parametrize("swapped", [False, True])
def test_swiglu_one_tensor_and_fused_pack(zest_gpu, oracle, swapped):
    # one tensor [rows][2f]: gate and up are its halves (swapped: up first)
    rows, f = 2048, 9728
    x = Rng(70).normal(rows * 2 * f, 0, 1.5).reshape(rows, 2 * f)
    xt = _dev(x)
    g, u = (xt[:, f:], xt[:, :f]) if swapped else (xt[:, :f], xt[:, f:])
    packed = zest_gpu.empty_act(rows, f)
    got = _host(zest_gpu.glu(2, g, u, f, packed=packed))
    gh, uh = (x[:, f:], x[:, :f]) if swapped else (x[:, :f], x[:, f:])
    assert nrmse(got, oracle.glu(2, gh, uh)) <= EXACT
    pk = zest_gpu.expanded_to_rows(_host(packed), rows, f)
    assert np.array_equal(pk.view(np.uint32), oracle.decode_rows(oracle.encode_rows(got)).view(np.uint32))


def test_add_mul_scale(zest_gpu, oracle):
    rows, d = 8, 256
    a = Rng(80).normal(rows * d, 0, 1.5).reshape(rows, d)
    b = Rng(81).normal(rows * d, 0, 1.5).reshape(rows, d)
    r = Rng(82).normal(d, 0, 1.5)
    assert nrmse(_host(zest_gpu.add(_dev(a), _dev(b))), oracle.add(a, b)) <= EXACT
    assert nrmse(_host(zest_gpu.add(_dev(a), _dev(r), b_is_row=True)), oracle.add_row(a, r)) <= EXACT
    assert nrmse(_host(zest_gpu.mul_row(_dev(a), _dev(r))), oracle.mul_row(a, r)) <= EXACT
    assert nrmse(_host(zest_gpu.scale(_dev(a), 0.37, 0.25)), oracle.scale(a, np.float32(0.37), np.float32(0.25))) <= EXACT


@pytest.mark.parametrize("rows,d,off", [(3, 7, 0), (5, 1030, 1), (70000, 8, 0), (2, 4096, 3), (4, 1028, 2)])
def test_add_mul_scale_odd_shapes(zest_gpu, oracle, rows, d, off):
    # widths that are not a multiple of 4, and operands starting `off` floats
    # past 16-byte alignment, take the scalar path; more rows than one grid
    # dimension holds (70000) are walked in a loop
    import torch
    n = rows * d
    a, b = Rng(83).normal(n + off, 0, 1.5), Rng(84).normal(n + off, 0, 1.5)
    r = Rng(85).normal(d + off, 0, 1.5)
    ta, tb, tr = (_dev(v)[off:] for v in (a, b, r))
    a2, b2, r2 = a[off:].reshape(rows, d), b[off:].reshape(rows, d), r[off:]
    assert np.array_equal(_host(zest_gpu.add(ta.view(rows, d), tb.view(rows, d))), oracle.add(a2, b2))
    assert np.array_equal(_host(zest_gpu.add(ta.view(rows, d), tr, b_is_row=True)), oracle.add_row(a2, r2))
    assert np.array_equal(_host(zest_gpu.mul_row(ta.view(rows, d), tr)), oracle.mul_row(a2, r2))
    assert nrmse(_host(zest_gpu.scale(ta, 0.37, 0.25)), oracle.scale(a[off:], np.float32(0.37), np.float32(0.25))) <= EXACT
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    zest_gpu.check_finite(ta.view(rows, d), flag)
    assert int(flag.item()) == 0
    bad = ta.clone().view(rows, d)
    bad[rows - 1, d - 1] = float("inf")
    zest_gpu.check_finite(bad, flag)
    assert int(flag.item()) == 1


ROPE_CASES = [  # (n_dims, mode, n_ctx_orig, freq_scale, ext_factor, factors): tests/test-host-ops.cpp:146-152
    (64, 0, 0, 1.0, 0.0, False), (64, 2, 0, 1.0, 0.0, False), (32, 0, 0, 1.0, 0.0, False),
    (48, 2, 0, 1.0, 0.0, False), (64, 2, 4096, 0.25, 1.0, False), (64, 2, 4096, 1.0, 0.0, True),
    (64, 0, 4096, 0.25, 1.0, True),
]


@pytest.mark.parametrize("n_dims,mode,n_ctx,fs,ext,factors", ROPE_CASES)
def test_rope(zest_gpu, oracle, n_dims, mode, n_ctx, fs, ext, factors):
    T, H, HD = 8, 4, 64
    x = Rng(90).normal(T * H * HD, 0, 1.5).reshape(T, H, HD)
    pos = (5000 + 300 * np.arange(T)).astype(np.int32)
    ff = (1.0 + 3.0 * Rng(91).uniform(n_dims // 2)).astype(np.float32) if factors else None
    want = oracle.rope(x, pos, ff, n_dims, mode, n_ctx, 10000.0, fs, ext, 1.0, 32.0, 1.0)
    corr = oracle.corr_dims(n_dims, n_ctx, 10000.0, 32.0, 1.0)
    got = zest_gpu.rope(_dev(x), _dev(pos), None if ff is None else _dev(ff), n_dims, mode, 10000.0, fs, ext, 1.0,
                        corr)
    assert nrmse(_host(got), want) <= EXACT


def test_rope_yarn_at_long_positions(zest_gpu, oracle):
    # positions of a 40k-token context with YaRN: the angle in the ramp
    # between the correction dimensions is a blend the CPU rounds step by
    # step; fusing it into a multiply-add moved the angle by an ulp, which at
    # these positions put the rotation 1.6e-5 off in nrmse (over the bar)
    T, H, HD = 31, 2, 128
    x = Rng(92).normal(T * H * HD, 0, 1.5).reshape(T, H, HD)
    pos = np.array([13575, 36435, 23620, 23342, 38472, 37492, 38234, 8472] * 4, dtype=np.int32)[:T]
    for mode in (0, 2):
        want = oracle.rope(x, pos, None, 128, mode, 4096, 10000.0, 0.25, 1.0, 1.0, 32.0, 1.0)
        corr = oracle.corr_dims(128, 4096, 10000.0, 32.0, 1.0)
        got = zest_gpu.rope(_dev(x), _dev(pos), None, 128, mode, 10000.0, 0.25, 1.0, 1.0, corr)
        assert nrmse(_host(got), want) <= 1e-6, mode


def _padding_is_zero(z, buf, rows, d):
    """The expanded operand's rows past `rows` and columns past d are zero."""
    full = z.expanded_to_rows(buf, z.rows_pad(rows), z.k_pad(d))
    return not full[rows:].any() and not full[:, d:].any()


@pytest.mark.parametrize("rows,d", [(5, 200), (300, 2560)])
def test_fused_packs_zero_their_padding(zest_gpu, oracle, rows, d):
    # the GEMM reads the operand up to its padded row count: the norm and GLU
    # packs write those rows (and the K padding) as zeros, whatever the
    # buffer held before
    import torch
    x = Rng(rows * 3 + d).normal(rows * d, 0, 1.5).reshape(rows, d)
    packed = zest_gpu.empty_act(rows, d)
    packed.fill_(0xFF)
    y = zest_gpu.rms_norm(_dev(x), 1e-6, packed=packed)
    host = _host(packed)
    assert _padding_is_zero(zest_gpu, host, rows, d)
    got = _host(y)
    assert np.array_equal(zest_gpu.expanded_to_rows(host, rows, d).view(np.uint32),
                          oracle.decode_rows(oracle.encode_rows(got)).view(np.uint32))
    g = Rng(rows + 1).normal(rows * d, 0, 1.5).reshape(rows, d)
    u = Rng(rows + 2).normal(rows * d, 0, 1.5).reshape(rows, d)
    packed.fill_(0xFF)
    h = zest_gpu.glu(2, _dev(g), _dev(u), d, packed=packed)
    host = _host(packed)
    assert _padding_is_zero(zest_gpu, host, rows, d)
    assert np.array_equal(zest_gpu.expanded_to_rows(host, rows, d).view(np.uint32),
                          oracle.decode_rows(oracle.encode_rows(_host(h))).view(np.uint32))
    del torch


def test_expanded_writers_random_shapes(zest_gpu, oracle):
    # every kernel that writes the expanded operand, over seeded odd shapes
    # (rows across 32-row sub-tile groups and 256-row padding, widths in steps
    # of 8 across 16- and 64-column boundaries), into buffers that held
    # garbage: the values are the oracle's encoding of each kernel's fp32
    # result and the padding is zero
    import torch
    rng = np.random.default_rng(31)
    for _ in range(10):
        rows = int(rng.choice([1, 31, 33, 95, 257, 300, 700]))
        d = int(rng.integers(1, 200)) * 8
        x = rng.normal(0, 1.5, (rows, d)).astype(np.float32)
        want = oracle.decode_rows(oracle.encode_rows(x)).view(np.uint32)
        buf = zest_gpu.empty_act(rows, d)
        buf.fill_(0xFF)
        zest_gpu.pack_act_x(_dev(x), out=buf)
        host = _host(buf)
        assert np.array_equal(zest_gpu.expanded_to_rows(host, rows, d).view(np.uint32), want), (rows, d)
        assert _padding_is_zero(zest_gpu, host, rows, d), (rows, d)
        ex = zest_gpu.expand_act(zest_gpu.pack_act(_dev(x)), rows, d)
        assert np.array_equal(_host(ex), host), (rows, d)
        buf.fill_(0xFF)
        y = _host(zest_gpu.rms_norm(_dev(x), 1e-6, packed=buf))
        host = _host(buf)
        assert np.array_equal(zest_gpu.expanded_to_rows(host, rows, d).view(np.uint32),
                              oracle.decode_rows(oracle.encode_rows(y)).view(np.uint32)), (rows, d)
        assert _padding_is_zero(zest_gpu, host, rows, d), (rows, d)
        u = rng.normal(0, 1.5, (rows, d)).astype(np.float32)
        buf.fill_(0xFF)
        h = _host(zest_gpu.glu(2, _dev(x), _dev(u), d, packed=buf))
        host = _host(buf)
        assert np.array_equal(zest_gpu.expanded_to_rows(host, rows, d).view(np.uint32),
                              oracle.decode_rows(oracle.encode_rows(h)).view(np.uint32)), (rows, d)
        assert _padding_is_zero(zest_gpu, host, rows, d), (rows, d)
    del torch

