"""GGUF quantisers for synthetic weights (what ggml_quantize_chunk is to the
reference's tests, tests/test-mul-mat.cpp:174): valid Q8_0 and Q4_K rows
built from float weights, with torch ops so they run on the CPU or the GPU.

The bytes they produce are the shared input of every path (GPU converter,
CPU oracle, CPU baseline), so they need not reproduce ggml's own quantiser
search; they follow the public block formats exactly:
  Q8_0  34 bytes / 32 values: fp16 d = absmax/127, then 32 int8 round(x/d)
  Q4_K 144 bytes / 256 values: fp16 d, fp16 dmin, 12 bytes of 6-bit
        (scale, min) pairs for the 8 sub-blocks of 32, 128 bytes of nibbles
        (group j of 64: low nibbles = values 64j..64j+31, high = the next 32)
"""
from __future__ import annotations

import torch


def _fp16_bytes(v: torch.Tensor) -> torch.Tensor:
    """float tensor [...] -> its fp16 (RNE) bytes [..., 2], little-endian."""
    return v.to(torch.float16).contiguous().view(torch.uint8).reshape(*v.shape, 2)


def quantize_q8_0(w: torch.Tensor) -> torch.Tensor:
    """w float32 [N][K] (K % 32 == 0) -> uint8 [N][K/32*34]."""
    n, k = w.shape
    b = w.float().reshape(n, k // 32, 32)
    amax = b.abs().amax(dim=2)
    d = amax / 127.0
    d16 = d.to(torch.float16)
    inv = torch.where(d > 0, 1.0 / d, torch.zeros_like(d))
    x = b * inv[..., None]
    q = torch.sign(x) * torch.floor(x.abs() + 0.5)  # roundf: half away from zero
    q = q.clamp(-128, 127).to(torch.int8)
    out = torch.empty((n, k // 32, 34), dtype=torch.uint8, device=w.device)
    out[..., :2] = d16.contiguous().view(torch.uint8).reshape(n, k // 32, 2)
    out[..., 2:] = q.view(torch.uint8)
    return out.reshape(n, k // 32 * 34)


def quantize_q4_k(w: torch.Tensor) -> torch.Tensor:
    """w float32 [N][K] (K % 256 == 0) -> uint8 [N][K/256*144].

    Per sub-block of 32: min m = max(0, -min(x)), scale s = (max(x) + m)/15;
    per super-block d = max(s)/63, dmin = max(m)/63 (as fp16); 6-bit
    sc = round(s/d), mn = round(m/dmin); q = round((x + dmin*mn)/(d*sc)) in 0..15.
    """
    n, k = w.shape
    nb = k // 256
    x = w.float().reshape(n, nb, 8, 32)
    mn = torch.clamp(-x.amin(dim=3), min=0.0)
    mx = x.amax(dim=3)
    s = torch.clamp((mx + mn) / 15.0, min=0.0)
    d = (s.amax(dim=2) / 63.0).to(torch.float16)
    dmin = (mn.amax(dim=2) / 63.0).to(torch.float16)
    df, dminf = d.float(), dmin.float()
    sc = torch.where(df[..., None] > 0, torch.round(s / df[..., None].clamp(min=1e-30)), torch.zeros_like(s))
    sc = sc.clamp(0, 63)
    mq = torch.where(dminf[..., None] > 0, torch.round(mn / dminf[..., None].clamp(min=1e-30)), torch.zeros_like(mn))
    mq = mq.clamp(0, 63)
    step = df[..., None] * sc                      # [n, nb, 8]
    offs = dminf[..., None] * mq
    q = torch.where(step[..., None] > 0, torch.round((x + offs[..., None]) / step[..., None].clamp(min=1e-30)),
                    torch.zeros_like(x))
    q = q.clamp(0, 15).to(torch.uint8)             # [n, nb, 8, 32]

    sci, mi = sc.to(torch.uint8), mq.to(torch.uint8)
    scales = torch.empty((n, nb, 12), dtype=torch.uint8, device=w.device)
    scales[..., 0:4] = sci[..., 0:4] | ((sci[..., 4:8] >> 4) << 6)
    scales[..., 4:8] = mi[..., 0:4] | ((mi[..., 4:8] >> 4) << 6)
    scales[..., 8:12] = (sci[..., 4:8] & 0xF) | ((mi[..., 4:8] & 0xF) << 4)
    qs = (q[:, :, 0::2, :] | (q[:, :, 1::2, :] << 4)).reshape(n, nb, 128)

    out = torch.empty((n, nb, 144), dtype=torch.uint8, device=w.device)
    out[..., 0:2] = _fp16_bytes(d)
    out[..., 2:4] = _fp16_bytes(dmin)
    out[..., 4:16] = scales
    out[..., 16:] = qs
    return out.reshape(n, nb * 144)


def quantize(wtype: int, w: torch.Tensor) -> torch.Tensor:
    if wtype == 8:
        return quantize_q8_0(w)
    if wtype == 12:
        return quantize_q4_k(w)
    if wtype == 0:
        return w.float().contiguous().view(torch.uint8).reshape(w.shape[0], -1)
    raise ValueError(f"no quantiser for type {wtype}")
