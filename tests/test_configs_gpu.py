"""The BASELINE configurations on the GPU against the oracle, at their real
shapes (the reference exercises its backend over a shape list,
tests/test-mul-mat.cpp:101-125 and :140-157, and end to end on models).

* Configuration 5 (27B-class, hidden 5120, all Q4_K, 4096-token chunk, 0.5% of
  channels x30): each distinct launch of a layer, the q/k/v group, O plus the
  residual, the fused gate/up GEMM and down plus the residual.
* Configuration 4 (hidden 1024, Q8_0, FFN 1024 -> 4096 -> 1024): the same
  launches at every chunk the dispatch gate claims (1024, 1536 and 4096
  tokens; it declines 256 and 512, which tests/cpp/test_dispatch_gate.cpp
  checks).
* Configuration 3 (Qwen3-4B-shaped): two layers chained at a 2048-token chunk,
  the residual stream carried from launch to launch and layer to layer.
* Configuration 2 (the SwiGLU triple, Q4_K, 1% of channels x20): fused
  gate/up -> packed SwiGLU -> down as one chain.

Matmuls meet the GEMM bar against fp64 sums over the same decoded operands on
sampled rows: |g - r64| <= 2 K 2^-24 sum|a b| (the products are exact, so
only the fp32 summation order may differ, and any order stays inside this),
with one more rounding where a residual is added; the max relative error
over outputs not near zero must also be under the north star's 1e-3.
Scaling the activations by 4 shifts every exponent byte, and every output
must scale exactly (checked on all rows).
Packed operands are bit-exact with the oracle's encoder; the GLU meets the
host ops' bar (nrmse <= 1e-5, tests/test-host-ops.cpp:79).
"""
from __future__ import annotations

import numpy as np
import pytest
from helpers import load_quant, nrmse

pytestmark = pytest.mark.gpu

Q4_K, Q8_0 = 12, 8
SWIGLU = 2


def _gen(seed):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def _acts(m, k, seed, outlier_frac=0.0, outlier_scale=1.0):
    """fp32 N(0,1) activations [m][k] on the GPU, a fraction of the channels scaled."""
    import torch
    g = _gen(seed)
    x = torch.randn((m, k), generator=g, device="cuda")
    if outlier_frac > 0:
        ch = torch.randperm(k, generator=g, device="cuda")[:max(1, int(k * outlier_frac))]
        x[:, ch] *= outlier_scale
    return x


def _raw(wtype, n, k, seed):
    """GGUF rows of N(0, 0.02) weights, quantised on the GPU."""
    import torch
    w = torch.randn((n, k), generator=_gen(seed), device="cuda") * 0.02
    return load_quant().quantize(wtype, w)


def _rows(m, n=24):
    return np.unique(np.concatenate([np.linspace(0, m - 1, n).astype(int), [m - 1]]))


def _wdec(z, oracle, packed, n, k):
    return oracle.decode_rows(z.tiles_to_blocks(packed.cpu().numpy(), n, k))


def _adec(z, a, m, k, rows):
    return z.expanded_to_rows(a.cpu().numpy(), m, k)[rows]


def _check(got, r64, ab, k, res=None):
    """The GEMM bar on sampled rows; with `res`, got = acc + res rounded once more."""
    got = got.astype(np.float64)
    slack = 0.0
    if res is not None:
        slack = np.abs(got) * 2.0 ** -24
        got = got - res.astype(np.float64)
    err = np.abs(got - r64)
    bound = 2.0 * k * 2.0 ** -24 * ab + slack
    assert np.isfinite(got).all()
    ratio = float((err / np.maximum(bound, 1e-300)).max())
    assert ratio <= 1.0, ratio
    big = np.abs(r64) >= 1e-2 * np.sqrt((r64 ** 2).mean())
    maxrel = float((err[big] / np.abs(r64[big])).max())
    assert maxrel <= 1e-3, maxrel
    return ratio, maxrel


def _pack_check(z, oracle, x, a, rows):
    """The expanded operand's sampled rows are the oracle's encoding of x."""
    m, k = x.shape
    xs = x[rows].cpu().numpy()
    got = _adec(z, a, m, k, rows)
    assert np.array_equal(got.view(np.uint32), oracle.decode_rows(oracle.encode_rows(xs)).view(np.uint32))
    return got


def _nf():
    import torch
    return torch.zeros(1, dtype=torch.int32, device="cuda")


def qkv_group(z, oracle, m, hidden, ns, wtype, seed, outlier_frac=0.0, outlier_scale=1.0):
    import torch
    x = _acts(m, hidden, seed, outlier_frac, outlier_scale)
    a = z.pack_act_x(x)
    ws = [z.convert_weight(wtype, _raw(wtype, n, hidden, seed + 1 + i), n, hidden) for i, n in enumerate(ns)]
    nf = _nf()
    outs = z.gemm_group(a, m, ws, ns, hidden, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    rows = _rows(m)
    ad = _pack_check(z, oracle, x, a, rows)
    for i, n in enumerate(ns):
        r64, ab = oracle.mul_mat_f64(_wdec(z, oracle, ws[i], n, hidden), ad)
        _check(outs[i].cpu().numpy()[rows], r64, ab, hidden)
    # x * 4: every activation exponent byte + 2, every output exactly x 4
    outs4 = z.gemm_group(z.pack_act_x(x * 4.0), m, ws, ns, hidden)
    for o, o4 in zip(outs, outs4):
        assert torch.equal(o4, o * 4.0)


def proj_residual(z, oracle, m, n, k, wtype, seed, outlier_frac=0.0, outlier_scale=1.0):
    """h = h + A . W^T in place (O and down), then the shift property on the plain GEMM."""
    import torch
    x = _acts(m, k, seed, outlier_frac, outlier_scale)
    a = z.pack_act_x(x)
    wp = z.convert_weight(wtype, _raw(wtype, n, k, seed + 1), n, k)
    h0 = _acts(m, n, seed + 2)
    h = h0.clone()
    nf = _nf()
    z.gemm_residual(a, m, wp, n, k, h, out=h, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    rows = _rows(m)
    ad = _pack_check(z, oracle, x, a, rows)
    r64, ab = oracle.mul_mat_f64(_wdec(z, oracle, wp, n, k), ad)
    _check(h.cpu().numpy()[rows], r64, ab, k, res=h0.cpu().numpy()[rows])
    c = z.gemm(a, m, wp, n, k)
    c4 = z.gemm(z.pack_act_x(x * 4.0), m, wp, n, k)
    torch.cuda.synchronize()
    assert torch.equal(c4, c * 4.0)


def gate_up(z, oracle, m, f, k, wtype, seed, outlier_frac=0.0, outlier_scale=1.0):
    """The fused gate/up GEMM: h = SiLU(g) u and its packed operand."""
    import torch
    x = _acts(m, k, seed, outlier_frac, outlier_scale)
    a = z.pack_act_x(x)
    gate, up = _raw(wtype, f, k, seed + 1), _raw(wtype, f, k, seed + 2)
    wgu = z.convert_weight_gu(wtype, gate, up, f, k)
    nf = _nf()
    xo, h = z.gemm_glu(SWIGLU, a, m, wgu, f, k, h=True, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    rows = _rows(m)
    ad = _pack_check(z, oracle, x, a, rows)
    hs = h.cpu().numpy()[rows]
    # the operand is the encoding of h
    xd = z.expanded_to_rows(xo.cpu().numpy(), m, f)[rows]
    assert np.array_equal(xd.view(np.uint32), oracle.decode_rows(oracle.encode_rows(hs)).view(np.uint32))
    # h against the oracle's SwiGLU of fp64 gate and up products over the
    # same decoded operands (the gate and up rows converted on their own)
    g64, _ = oracle.mul_mat_f64(_wdec(z, oracle, z.convert_weight(wtype, gate, f, k), f, k), ad)
    u64, _ = oracle.mul_mat_f64(_wdec(z, oracle, z.convert_weight(wtype, up, f, k), f, k), ad)
    want = oracle.glu(SWIGLU, g64.astype(np.float32), u64.astype(np.float32))
    assert nrmse(hs, want) <= 1e-5


# ---- configuration 2: the SwiGLU MUL_MAT triple ---------------------------------------------

def test_config2_swiglu_triple(zest_gpu, oracle):
    """BASELINE configuration 2 as one chain: 2048 tokens of N(0,1) with 1% of
    the channels x20 -> the fused gate/up GEMM (Q4_K, 2560 -> 2 x 9728) ->
    its SwiGLU, packed by its epilogue -> down (Q4_K, 9728 -> 2560). Every
    stage is checked on sampled rows against the oracle on that stage's own
    GPU input: the packs bit-exact with the oracle's encoder, the gate and up
    sums (the fused launch's are those of the plain GEMM over the interleaved
    weight, bit for bit) and the down projection within the GEMM bar with no
    relative slack, and h within the host ops' bar of the oracle's SwiGLU."""
    import torch
    z = zest_gpu
    m, H, F = 2048, 2560, 9728
    x = _acts(m, H, 201, outlier_frac=0.01, outlier_scale=20.0)
    a = z.pack_act_x(x)
    gate, up = _raw(Q4_K, F, H, 202), _raw(Q4_K, F, H, 203)
    wgu = z.convert_weight_gu(Q4_K, gate, up, F, H)
    wdn = z.convert_weight(Q4_K, _raw(Q4_K, H, F, 204), H, F)
    nf = _nf()
    xo, h = z.gemm_glu(SWIGLU, a, m, wgu, F, H, h=True, nonfinite=nf)
    y = z.gemm(xo, m, wdn, H, F, nonfinite=nf)
    c = z.gemm(a, m, wgu, 2 * F, H).view(m, F // 32, 2, 32)
    g = c[:, :, 0, :].reshape(m, F).contiguous()
    u = c[:, :, 1, :].reshape(m, F).contiguous()
    h_chain = z.glu(SWIGLU, g, u, F)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    assert torch.equal(h.view(torch.int32), h_chain.view(torch.int32))
    rows = _rows(m)
    ad = _pack_check(z, oracle, x, a, rows)
    # gate and up against fp64 sums over the same decoded operands
    g64, gab = oracle.mul_mat_f64(_wdec(z, oracle, z.convert_weight(Q4_K, gate, F, H), F, H), ad)
    u64, uab = oracle.mul_mat_f64(_wdec(z, oracle, z.convert_weight(Q4_K, up, F, H), F, H), ad)
    _check(g.cpu().numpy()[rows], g64, gab, H)
    _check(u.cpu().numpy()[rows], u64, uab, H)
    hs = h.cpu().numpy()[rows]
    e = nrmse(hs, oracle.glu(SWIGLU, g64.astype(np.float32), u64.astype(np.float32)))
    assert e <= 1e-5, e
    # the down projection's operand is the encoding of h, and its product
    dd = z.expanded_to_rows(xo.cpu().numpy(), m, F)[rows]
    assert np.array_equal(dd.view(np.uint32), oracle.decode_rows(oracle.encode_rows(hs)).view(np.uint32))
    r64, ab = oracle.mul_mat_f64(_wdec(z, oracle, wdn, H, F), dd)
    ratio, maxrel = _check(y.cpu().numpy()[rows], r64, ab, F)
    print(f"config 2 triple: down bound use {ratio:.2f}, max rel {maxrel:.2e}, SwiGLU nrmse {e:.2e}")


# ---- configuration 5: 27B-class layer at a 4096-token chunk --------------------------------

C5 = dict(m=4096, outlier_frac=0.005, outlier_scale=30.0)


def test_config5_qkv_group(zest_gpu, oracle):
    qkv_group(zest_gpu, oracle, hidden=5120, ns=[6144, 1024, 1024], wtype=Q4_K, seed=501, **C5)


def test_config5_o_residual(zest_gpu, oracle):
    proj_residual(zest_gpu, oracle, n=5120, k=6144, wtype=Q4_K, seed=502, **C5)


def test_config5_gate_up_fused(zest_gpu, oracle):
    gate_up(zest_gpu, oracle, f=17408, k=5120, wtype=Q4_K, seed=503, **C5)


def test_config5_down_residual(zest_gpu, oracle):
    proj_residual(zest_gpu, oracle, n=5120, k=17408, wtype=Q4_K, seed=504, **C5)


# ---- configuration 4: hidden 1024, Q8_0, every claimed chunk -------------------------------

@pytest.mark.parametrize("m", [1024, 1536, 4096])
def test_config4_layer_launches(zest_gpu, oracle, m):
    z = zest_gpu
    qkv_group(z, oracle, m, hidden=1024, ns=[1024, 1024, 1024], wtype=Q8_0, seed=400 + m)
    proj_residual(z, oracle, m, n=1024, k=1024, wtype=Q8_0, seed=410 + m)
    gate_up(z, oracle, m, f=4096, k=1024, wtype=Q8_0, seed=420 + m)
    proj_residual(z, oracle, m, n=1024, k=4096, wtype=Q8_0, seed=430 + m)


# ---- configuration 3: two Qwen3-4B-shaped layers chained ---------------------------------

def test_config3_two_layers_chained(zest_gpu, oracle):
    """Stack.run_chunk over two layers at 2048 tokens, then the same chain
    stage by stage: every stage is checked against the oracle on its own
    (GPU) input, and the stage-by-stage chain must reproduce run_chunk's
    result bit for bit. The rows are independent (attention is excluded: the
    O input is the Q output), so the checks use sampled rows. Finally the
    whole chain against the oracle's chain from the same x (every pack
    applied, every GEMM summed in fp64 on the CPU), normwise: two faithful
    chains part wherever a norm's output differs in its last bit (the GPU
    reduces the sum of squares in another order), since that can flip the
    bfp16 rounding of a packed value, and the flips grow through the GLU and
    the layers. Calibrated on the CPU: scaling each row of the oracle's own
    norm output by 1 +- 2^-22 (2 ulp) moves its two-layer chain by nrmse
    3.8e-3 (1 ulp: 0); summing the GEMMs in fp32 instead of fp64 moves it by
    5e-9. The bar is the reference's accuracy scale for its NPU path against
    fp64, 1e-2 (docs/results/lemonade-clean-build-ctest.txt:282-283); any
    structural error (a wrong weight, a lost residual) is of order 1."""
    import torch
    import ggml_xdna_amd.stack as st
    z = zest_gpu
    cfg = st.StackConfig("qwen3-4b-2", 2, 2560, 4096, 1024, 9728, Q4_K, Q8_0, Q4_K, Q8_0, 2048, 2048)
    s = st.Stack(cfg, seed=3)
    x = s.x[:2048]
    h_run = s.run_chunk(x).clone()
    torch.cuda.synchronize()

    m, H, eps = 2048, cfg.hidden, 1e-6
    rows = _rows(m, 16)
    h = x.clone()
    hc = x.cpu().numpy()[rows].astype(np.float32)   # the oracle's own chain
    for L in s.layers:
        w = {name: _wdec(z, oracle, L.w[name], n, k) for name, n, k, _ in cfg.matmuls()
             if name in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_down")}
        wgu = _wdec(z, oracle, L.w["ffn_gate_up"], 2 * cfg.ffn, H)
        # interleaved by 32-row groups: gate rows, then the up rows that pair with them
        wgu = wgu.reshape(cfg.ffn // 32, 2, 32, H)
        w["ffn_gate"] = wgu[:, 0].reshape(cfg.ffn, H)
        w["ffn_up"] = wgu[:, 1].reshape(cfg.ffn, H)
        an, fn = L.attn_norm.cpu().numpy(), L.ffn_norm.cpu().numpy()

        # RMSNorm * w_attn, packed
        y = z.rms_norm(h, eps, L.attn_norm, y=True, packed=s.pa)
        torch.cuda.synchronize()
        hs = h.cpu().numpy()[rows]
        ys = y.cpu().numpy()[rows]
        assert nrmse(ys, oracle.mul_row(oracle.rms_norm(hs, eps), an)) <= 1e-5
        ad = _pack_check(z, oracle, y, s.pa, rows)
        # q, k, v
        qo, ko, vo = z.gemm_group(s.pa, m, [L.w["attn_q"], L.w["attn_k"], L.w["attn_v"]],
                                  [cfg.q, cfg.kv, cfg.kv], H)
        for name, o in (("attn_q", qo), ("attn_k", ko), ("attn_v", vo)):
            r64, ab = oracle.mul_mat_f64(w[name], ad)
            _check(o.cpu().numpy()[rows], r64, ab, H)
        # O + residual, on Q's output as the stand-in attention output
        z.pack_act_x(qo, out=s.po)
        od = _pack_check(z, oracle, qo, s.po, rows)
        h_before = h.cpu().numpy()[rows]
        z.gemm_residual(s.po, m, L.w["attn_output"], H, cfg.q, h, out=h)
        r64, ab = oracle.mul_mat_f64(w["attn_output"], od)
        _check(h.cpu().numpy()[rows], r64, ab, cfg.q, res=h_before)
        # RMSNorm * w_ffn, packed
        y = z.rms_norm(h, eps, L.ffn_norm, y=True, packed=s.pa)
        hs = h.cpu().numpy()[rows]
        assert nrmse(y.cpu().numpy()[rows], oracle.mul_row(oracle.rms_norm(hs, eps), fn)) <= 1e-5
        ad = _pack_check(z, oracle, y, s.pa, rows)
        # fused gate/up -> SwiGLU -> packed
        _, hg = z.gemm_glu(SWIGLU, s.pa, m, L.w["ffn_gate_up"], cfg.ffn, H, xout=s.pd, h=True)
        g64, _ = oracle.mul_mat_f64(w["ffn_gate"], ad)
        u64, _ = oracle.mul_mat_f64(w["ffn_up"], ad)
        hgs = hg.cpu().numpy()[rows]
        assert nrmse(hgs, oracle.glu(SWIGLU, g64.astype(np.float32), u64.astype(np.float32))) <= 1e-5
        dd = z.expanded_to_rows(s.pd.cpu().numpy(), m, cfg.ffn)[rows]
        assert np.array_equal(dd.view(np.uint32), oracle.decode_rows(oracle.encode_rows(hgs)).view(np.uint32))
        # down + residual
        h_before = h.cpu().numpy()[rows]
        z.gemm_residual(s.pd, m, L.w["ffn_down"], H, cfg.ffn, h, out=h)
        r64, ab = oracle.mul_mat_f64(w["ffn_down"], dd)
        _check(h.cpu().numpy()[rows], r64, ab, cfg.ffn, res=h_before)

        # the oracle's chain for the sampled rows, from its own values
        def mm(wm, xin):
            xq = oracle.decode_rows(oracle.encode_rows(xin))
            return oracle.mul_mat_f64(wm, xq)[0].astype(np.float32)
        a_in = oracle.mul_row(oracle.rms_norm(hc, eps), an)
        q_c = mm(w["attn_q"], a_in)
        hc = (hc.astype(np.float64) + mm(w["attn_output"], q_c)).astype(np.float32)
        f_in = oracle.mul_row(oracle.rms_norm(hc, eps), fn)
        hg_c = oracle.glu(SWIGLU, mm(w["ffn_gate"], f_in), mm(w["ffn_up"], f_in))
        hc = (hc.astype(np.float64) + mm(w["ffn_down"], hg_c)).astype(np.float32)

    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int32), h_run.view(torch.int32)), "stage-by-stage chain differs from run_chunk"
    e = nrmse(h.cpu().numpy()[rows], hc)
    print(f"two-layer chain against the oracle's: nrmse {e:.2e}")
    assert e <= 1e-2, e
