"""Synthetic decoder-stack workloads of the prefill MUL_MAT path (the
BASELINE configurations), run through the C ABI on one GPU.

A layer, for one chunk of M tokens with residual stream h [M][H] (fp32):
    RMS_NORM(h) * w_attn   -> packed (fused)        xdna-exec's norm -> q/k/v piece
    Q, K, V = GEMM(packed, Wq / Wk / Wv)            one grouped launch
    (attention is excluded; the O projection's input is a stand-in: Q's output)
    pack(Q) ; h = h + GEMM(., Wo)                   the residual add in the GEMM's store
    RMS_NORM(h) * w_ffn    -> packed (fused)
    SiLU(packed . Wgate) * (packed . Wup) -> packed  one fused gate/up GEMM
                                                    (xdna-exec's find_fusions)
    h = h + GEMM(., Wdown)
With fused=False the gate and up are two GEMMs and the SwiGLU its own kernel,
as for a GLU that cannot be fused.
Weights are random-init N(0, 0.02), quantised to GGUF on the GPU, converted
once into the resident bfp16 cache (timed separately, as the reference
reports warm prefill with its one-time copy build apart).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import ggml_xdna_amd as z
from ggml_xdna_amd import quant

BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk
HBM_PEAK_GBS = 8000.0


@dataclass
class StackConfig:
    name: str
    layers: int
    hidden: int
    q: int
    kv: int
    ffn: int
    qkv_type: int     # GGUF type of Q/K/V (and gate/up)
    o_type: int
    ffn_type: int     # gate/up
    down_type: int
    tokens: int       # prompt length
    chunk: int        # tokens per chunk
    outlier_frac: float = 0.0
    outlier_scale: float = 1.0

    def matmuls(self):
        """(name, N, K, type) of one layer's weights."""
        return [("attn_q", self.q, self.hidden, self.qkv_type), ("attn_k", self.kv, self.hidden, self.qkv_type),
                ("attn_v", self.kv, self.hidden, self.qkv_type), ("attn_output", self.hidden, self.q, self.o_type),
                ("ffn_gate", self.ffn, self.hidden, self.ffn_type), ("ffn_up", self.ffn, self.hidden, self.ffn_type),
                ("ffn_down", self.hidden, self.ffn, self.down_type)]

    def flops_per_token(self) -> float:
        return 2.0 * sum(n * k for _, n, k, _ in self.matmuls()) * self.layers


CONFIGS = {
    # Qwen3-4B-shaped, 36 layers, 8192 tokens in 2048-token chunks
    "qwen3-4b": StackConfig("qwen3-4b", 36, 2560, 4096, 1024, 9728, z.TYPE_Q4_K, z.TYPE_Q8_0, z.TYPE_Q4_K,
                            z.TYPE_Q8_0, 8192, 2048),
    # hidden 1024, 16 layers, Q8_0, chunk swept by the caller
    "small-1024": StackConfig("small-1024", 16, 1024, 1024, 1024, 4096, z.TYPE_Q8_0, z.TYPE_Q8_0, z.TYPE_Q8_0,
                              z.TYPE_Q8_0, 4096, 4096),
    # 27B-class, 64 layers, all Q4_K, one 4096-token chunk, 0.5% outliers x30
    "dense-27b": StackConfig("dense-27b", 64, 5120, 6144, 1024, 17408, z.TYPE_Q4_K, z.TYPE_Q4_K, z.TYPE_Q4_K,
                             z.TYPE_Q4_K, 4096, 4096, 0.005, 30.0),
}


@dataclass
class Layer:
    w: dict = field(default_factory=dict)      # name -> packed bfp16 cache entry
    attn_norm: object = None
    ffn_norm: object = None


class Stack:
    """Weights resident in HBM plus per-chunk work buffers."""

    def __init__(self, cfg: StackConfig, seed: int = 0, device: str = "cuda", fused: bool = True, chunk=None):
        import torch
        self.cfg, self.device, self.fused = cfg, device, fused
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        self.layers: list[Layer] = []
        self.convert_bytes = 0.0   # algorithmic bytes of the one-time conversion
        self.convert_ms = 0.0
        raw_by_shape = {}
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for li in range(cfg.layers):
            L = Layer()
            for name, n, k, t in cfg.matmuls():
                key = (name, n, k, t)
                # distinct random weights per shape; layers share the GGUF source bytes
                # (values do not change the work) but each gets its own cache entry
                if key not in raw_by_shape:
                    w = torch.randn((n, k), generator=g, device=device) * 0.02
                    raw_by_shape[key] = quant.quantize(t, w)
                    del w
                if fused and name == "ffn_gate" and ("ffn_up", n, k, t) not in raw_by_shape:
                    w = torch.randn((n, k), generator=g, device=device) * 0.02
                    raw_by_shape[("ffn_up", n, k, t)] = quant.quantize(t, w)
                    del w
                raw = raw_by_shape[key]
                if fused and name == "ffn_up":
                    continue  # converted with the gate, below
                ev0.record()
                if fused and name == "ffn_gate":
                    up = raw_by_shape[("ffn_up", n, k, t)]
                    L.w["ffn_gate_up"] = z.convert_weight_gu(t, raw, up, n, k)
                    nbytes = raw.numel() + up.numel() + 2 * n * k * 9 / 8
                else:
                    L.w[name] = z.convert_weight(t, raw, n, k)
                    nbytes = raw.numel() + n * k * 9 / 8
                ev1.record()
                ev1.synchronize()
                self.convert_ms += ev0.elapsed_time(ev1)
                self.convert_bytes += nbytes
            L.attn_norm = 1.0 + 0.1 * torch.randn(cfg.hidden, generator=g, device=device)
            L.ffn_norm = 1.0 + 0.1 * torch.randn(cfg.hidden, generator=g, device=device)
            self.layers.append(L)
        del raw_by_shape
        self.chunk = chunk or cfg.chunk
        self._alloc(self.chunk)
        x = torch.randn((cfg.tokens, cfg.hidden), generator=g, device=device)
        if cfg.outlier_frac > 0:
            nout = max(1, int(cfg.hidden * cfg.outlier_frac))
            ch = torch.randperm(cfg.hidden, generator=g, device=device)[:nout]
            x[:, ch] *= cfg.outlier_scale
        self.x = x

    def _alloc(self, m: int):
        import torch
        c, dev = self.cfg, self.device
        f32 = dict(dtype=torch.float32, device=dev)
        self.h = torch.empty((m, c.hidden), **f32)
        self.qo = torch.empty((m, c.q), **f32)
        self.ko = torch.empty((m, c.kv), **f32)
        self.vo = torch.empty((m, c.kv), **f32)
        if not self.fused:
            self.go = torch.empty((m, c.ffn), **f32)
            self.uo = torch.empty((m, c.ffn), **f32)
        # the matmuls' activation operands (the bfp16 pack, expanded)
        self.pa = z.empty_act(m, c.hidden, dev)
        self.po = z.empty_act(m, c.q, dev)
        self.pd = z.empty_act(m, c.ffn, dev)

    def run_chunk(self, x_chunk, gemm_events=None):
        """One chunk through every layer. gemm_events: a list to which
        (start, end, flops) event pairs around each GEMM are appended."""
        import torch
        c, m = self.cfg, x_chunk.shape[0]
        eps = 1e-6
        # a short last chunk uses the first m rows of every buffer (the
        # packed operands are laid out for m rows by their writer and reader)
        h, qo, ko, vo = (t[:m] for t in (self.h, self.qo, self.ko, self.vo))
        go, uo = (self.go[:m], self.uo[:m]) if not self.fused else (None, None)
        h.copy_(x_chunk)

        def timed(fn, flops):
            if gemm_events is None:
                fn()
                return
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            gemm_events.append((e0, e1, flops))

        def gemm(a, wname, L, n, k, out):
            timed(lambda: z.gemm(a, m, L.w[wname], n, k, out=out), 2.0 * m * n * k)

        for L in self.layers:
            z.rms_norm(h, eps, L.attn_norm, y=None, packed=self.pa)
            # q, k and v share their input: one launch (the reference's group)
            timed(lambda: z.gemm_group(self.pa, m, [L.w["attn_q"], L.w["attn_k"], L.w["attn_v"]],
                                       [c.q, c.kv, c.kv], c.hidden, outs=[qo, ko, vo]),
                  2.0 * m * (c.q + 2 * c.kv) * c.hidden)
            z.pack_act_x(qo, out=self.po)
            timed(lambda: z.gemm_residual(self.po, m, L.w["attn_output"], c.hidden, c.q, h, out=h),
                  2.0 * m * c.hidden * c.q)
            z.rms_norm(h, eps, L.ffn_norm, y=None, packed=self.pa)
            if self.fused:
                timed(lambda: z.gemm_glu(z.GLU_SWIGLU, self.pa, m, L.w["ffn_gate_up"], c.ffn, c.hidden,
                                         xout=self.pd), 4.0 * m * c.ffn * c.hidden)
            else:
                gemm(self.pa, "ffn_gate", L, c.ffn, c.hidden, go)
                gemm(self.pa, "ffn_up", L, c.ffn, c.hidden, uo)
                z.glu(z.GLU_SWIGLU, go, uo, c.ffn, y=None, packed=self.pd)
            timed(lambda: z.gemm_residual(self.pd, m, L.w["ffn_down"], c.hidden, c.ffn, h, out=h),
                  2.0 * m * c.hidden * c.ffn)
        return h

    def run_gemms(self):
        """The GEMM launches of one prompt step, back to back and on the
        operands the last step left (the same shapes, tiles and splits): the
        GEMM kernel's own time, without the host ops between launches.
        Returns (launches, flops)."""
        c = self.cfg
        n, flops = 0, 0.0
        for t0 in range(0, c.tokens, self.chunk):
            m = min(self.chunk, c.tokens - t0)
            h, qo, ko, vo = (t[:m] for t in (self.h, self.qo, self.ko, self.vo))
            for L in self.layers:
                z.gemm_group(self.pa, m, [L.w["attn_q"], L.w["attn_k"], L.w["attn_v"]], [c.q, c.kv, c.kv],
                             c.hidden, outs=[qo, ko, vo])
                z.gemm_residual(self.po, m, L.w["attn_output"], c.hidden, c.q, h, out=h)
                if self.fused:
                    z.gemm_glu(z.GLU_SWIGLU, self.pa, m, L.w["ffn_gate_up"], c.ffn, c.hidden, xout=self.pd)
                    n += 3
                else:
                    z.gemm(self.pa, m, L.w["ffn_gate"], c.ffn, c.hidden, out=self.go[:m])
                    z.gemm(self.pa, m, L.w["ffn_up"], c.ffn, c.hidden, out=self.uo[:m])
                    n += 4
                z.gemm_residual(self.pd, m, L.w["ffn_down"], c.hidden, c.ffn, h, out=h)
                n += 1
                flops += 2.0 * m * ((c.q + 2 * c.kv) * c.hidden + c.hidden * c.q + 2 * c.ffn * c.hidden +
                                    c.hidden * c.ffn)
        return n, flops

    def run_prompt(self, gemm_events=None):
        for t0 in range(0, self.cfg.tokens, self.chunk):
            self.run_chunk(self.x[t0:t0 + self.chunk], gemm_events)
