"""Python handle on libggml-zest.so through its C ABI (include/zest_hip.h).

This is plumbing for tests and bench.py: every call goes straight to the HIP
kernels in the library, on torch's current stream, with device memory owned
by torch tensors. There is no fallback: if the library is not built, or a
call fails, a ZestError is raised.

Loaded as ``ggml_xdna_amd`` (the directory name has a hyphen):
    spec = importlib.util.spec_from_file_location("ggml_xdna_amd", ".../ggml-xdna_amd/__init__.py")
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libggml-zest.so"

TYPE_F32, TYPE_Q8_0, TYPE_Q4_K = 0, 8, 12
GLU_REGLU, GLU_GEGLU, GLU_SWIGLU, GLU_GEGLU_ERF, GLU_GEGLU_QUICK = 0, 1, 2, 3, 4

TILE_ROWS, TILE_K, TILE_MANT, TILE_BYTES, ROW_ALIGN = 16, 64, 1024, 1152, 256


class ZestError(RuntimeError):
    pass


_lib = None

_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_f = ctypes.c_float
_c_i = ctypes.c_int

# name -> (restype, argtypes), as declared in include/zest_hip.h
SIGNATURES = {
    "zest_init": (_c_i, [_c_i]),
    "zest_self_test": (_c_i, []),
    "zest_last_error": (ctypes.c_char_p, []),
    "zest_rows_pad": (_c_i64, [_c_i64]),
    "zest_k_pad": (_c_i64, [_c_i64]),
    "zest_bfp16_bytes": (ctypes.c_size_t, [_c_i64, _c_i64]),
    "zest_raw_row_bytes": (ctypes.c_size_t, [_c_i, _c_i64]),
    "zest_act_bytes": (ctypes.c_size_t, [_c_i64, _c_i64]),
    "zest_pack_act": (_c_i, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "zest_pack_act_x": (_c_i, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "zest_expand_act": (_c_i, [_c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "zest_convert_weight": (_c_i, [_c_i, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "zest_gemm": (_c_i, [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p]),
    "zest_gemm_residual": (_c_i, [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p]),
    "zest_gemm_group": (_c_i, [_c_p, _c_i64, _c_i64, _c_i, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "zest_gemm_group_noalloc": (_c_i, [_c_p, _c_i64, _c_i64, _c_i, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "zest_release_stream": (_c_i, [_c_p]),
    "zest_convert_weight_gu": (_c_i, [_c_i, _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "zest_gemm_glu": (_c_i, [_c_i, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p]),
    "zest_rms_norm": (_c_i, [_c_p, _c_i64, _c_i64, _c_f, _c_p, _c_p, _c_p, _c_p]),
    "zest_glu": (_c_i, [_c_i, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "zest_add": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_i, _c_p, _c_p]),
    "zest_mul_row": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p]),
    "zest_scale": (_c_i, [_c_p, _c_i64, _c_f, _c_f, _c_p, _c_p]),
    "zest_check_finite": (_c_i, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "zest_rope": (_c_i, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i, _c_i, _c_f, _c_f, _c_f, _c_f,
                         _c_f, _c_f, _c_p, _c_p]),
}


def lib() -> ctypes.CDLL:
    """The loaded library; raises ZestError if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ZestError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        l = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype, f.argtypes = res, args
        _lib = l
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        raise ZestError(f"{what} failed ({status}): {lib().zest_last_error().decode()}")


# ---- layout arithmetic (mirrors csrc/zest_layout.h) --------------------------

def rows_pad(rows: int) -> int:
    return (rows + ROW_ALIGN - 1) // ROW_ALIGN * ROW_ALIGN


def k_pad(k: int) -> int:
    return (k + TILE_K - 1) // TILE_K * TILE_K


def bfp16_bytes(rows: int, k: int) -> int:
    return rows_pad(rows) * k_pad(k) // 8 * 9


def act_bytes(rows: int, k: int) -> int:
    """Bytes of an expanded activation operand: 2 per value, padded."""
    return rows_pad(rows) * k_pad(k) * 2


def expanded_to_rows(buf: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Expanded operand bytes -> float32 [rows][k] (the bf16 values widened)."""
    rp, kp = rows_pad(rows), k_pad(k)
    # [64-column chunk][32-row group][16-column quarter][row][column]
    t = np.frombuffer(np.ascontiguousarray(buf).tobytes(), dtype=np.uint16).reshape(kp // 64, rp // 32, 4, 32, 16)
    full = t.transpose(1, 3, 0, 2, 4).reshape(rp, kp)
    return (full.astype(np.uint32) << 16).view(np.float32)[:rows, :k]


def tiles_to_blocks(buf: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Packed tile-layout bytes -> the reference's row-major blocks
    [rows][k/8][9] (exponent byte, then 8 mantissas), the bijection that
    maps our order onto bfp16_encode_block's output row by row."""
    rp, kp = rows_pad(rows), k_pad(k)
    t = np.asarray(buf, dtype=np.uint8).reshape(kp // TILE_K, rp // TILE_ROWS, TILE_BYTES)
    mant = t[:, :, :TILE_MANT].reshape(kp // TILE_K, rp // TILE_ROWS, TILE_ROWS, TILE_K)
    mant = mant.transpose(1, 2, 0, 3).reshape(rp, kp // 8, 8)
    exps = t[:, :, TILE_MANT:].reshape(kp // TILE_K, rp // TILE_ROWS, TILE_ROWS, 8)
    exps = exps.transpose(1, 2, 0, 3).reshape(rp, kp // 8, 1)
    return np.concatenate([exps, mant], axis=2)[:rows, : k // 8, :]


def blocks_to_tiles(blocks: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Inverse of tiles_to_blocks (padding as zero blocks)."""
    rp, kp = rows_pad(rows), k_pad(k)
    full = np.zeros((rp, kp // 8, 9), dtype=np.uint8)
    full[:rows, : k // 8] = np.asarray(blocks, dtype=np.uint8).reshape(rows, k // 8, 9)
    mant = full[:, :, 1:].reshape(rp // TILE_ROWS, TILE_ROWS, kp // TILE_K, TILE_K).transpose(2, 0, 1, 3)
    exps = full[:, :, 0].reshape(rp // TILE_ROWS, TILE_ROWS, kp // TILE_K, 8).transpose(2, 0, 1, 3)
    out = np.empty((kp // TILE_K, rp // TILE_ROWS, TILE_BYTES), dtype=np.uint8)
    out[:, :, :TILE_MANT] = mant.reshape(kp // TILE_K, rp // TILE_ROWS, TILE_MANT)
    out[:, :, TILE_MANT:] = exps.reshape(kp // TILE_K, rp // TILE_ROWS, 128)
    return out.reshape(-1)


def raw_row_bytes(wtype: int, k: int) -> int:
    return {TYPE_F32: 4 * k, TYPE_Q8_0: k // 32 * 34, TYPE_Q4_K: k // 256 * 144}[wtype]


# ---- torch-facing calls --------------------------------------------------------

def _torch():
    import torch
    return torch


def _stream():
    return ctypes.c_void_p(_torch().cuda.current_stream().cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def init(device: int = 0) -> None:
    check(lib().zest_init(device), "zest_init")


def self_test() -> None:
    check(lib().zest_self_test(), "zest_self_test")


def empty_packed(rows: int, k: int, device="cuda"):
    torch = _torch()
    return torch.empty(bfp16_bytes(rows, k), dtype=torch.uint8, device=device)


def empty_act(rows: int, k: int, device="cuda"):
    """Space for an expanded activation operand (the GEMM's A)."""
    torch = _torch()
    return torch.empty(act_bytes(rows, k), dtype=torch.uint8, device=device)


def pack_act(x, out=None):
    """fp32 [M][K] device tensor -> packed bfp16 (uint8 device tensor)."""
    torch = _torch()
    assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
    m, k = x.shape
    out = empty_packed(m, k, x.device) if out is None else out
    check(lib().zest_pack_act(_ptr(x), m, k, x.stride(0), _ptr(out), _stream()), "zest_pack_act")
    return out


def pack_act_x(x, out=None):
    """fp32 [M][K] device tensor -> the GEMM's expanded activation operand."""
    torch = _torch()
    assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
    m, k = x.shape
    out = empty_act(m, k, x.device) if out is None else out
    check(lib().zest_pack_act_x(_ptr(x), m, k, x.stride(0), _ptr(out), _stream()), "zest_pack_act_x")
    return out


def expand_act(packed, m: int, k: int, out=None):
    """Packed bfp16 activations -> the expanded operand."""
    out = empty_act(m, k, packed.device) if out is None else out
    check(lib().zest_expand_act(_ptr(packed), m, k, _ptr(out), _stream()), "zest_expand_act")
    return out


def convert_weight(wtype: int, raw, n: int, k: int, out=None):
    """GGUF weight bytes (uint8 device tensor, n rows) -> packed bfp16."""
    out = empty_packed(n, k, raw.device) if out is None else out
    check(lib().zest_convert_weight(wtype, _ptr(raw), n, k, _ptr(out), _stream()), "zest_convert_weight")
    return out


def gemm(a_packed, m: int, w_packed, n: int, k: int, out=None, nonfinite=None):
    """c[m][n] fp32 = A . W^T: a_packed the expanded activations (pack_act_x),
    w_packed a packed bfp16 weight (convert_weight)."""
    torch = _torch()
    out = torch.empty((m, n), dtype=torch.float32, device=a_packed.device) if out is None else out
    check(lib().zest_gemm(_ptr(a_packed), m, _ptr(w_packed), n, k, _ptr(out), out.stride(0), _ptr(nonfinite),
                          _stream()), "zest_gemm")
    return out


def gemm_residual(a_packed, m: int, w_packed, n: int, k: int, res, out=None, nonfinite=None):
    """c[m][n] = A . W^T + res (res may be out itself: an in-place residual add)."""
    torch = _torch()
    out = torch.empty((m, n), dtype=torch.float32, device=a_packed.device) if out is None else out
    check(lib().zest_gemm_residual(_ptr(a_packed), m, _ptr(w_packed), n, k, _ptr(res), res.stride(0), _ptr(out),
                                   out.stride(0), _ptr(nonfinite), _stream()), "zest_gemm_residual")
    return out


def gemm_group(a_packed, m: int, weights, ns, k: int, outs=None, nonfinite=None, noalloc=False):
    """Several weights sharing one activation operand in one launch:
    outs[i][m][ns[i]] = A . W_i^T. Returns the outputs. noalloc: through
    zest_gemm_group_noalloc (split-K workspace from the library's static
    array; the outputs must then be given)."""
    torch = _torch()
    n = len(weights)
    outs = [torch.empty((m, ni), dtype=torch.float32, device=a_packed.device) for ni in ns] if outs is None else outs
    P, I64 = ctypes.c_void_p * n, ctypes.c_int64 * n
    w = P(*[t.data_ptr() for t in weights])
    c = P(*[t.data_ptr() for t in outs])
    name = "zest_gemm_group_noalloc" if noalloc else "zest_gemm_group"
    check(getattr(lib(), name)(_ptr(a_packed), m, k, n, w, I64(*ns), c, I64(*[t.stride(0) for t in outs]),
                               _ptr(nonfinite), _stream()), name)
    return outs


def convert_weight_gu(wtype: int, gate, up, f: int, k: int, out=None):
    """A GLU's gate and up GGUF weights (uint8 device tensors, f rows each) ->
    one packed weight of 2f rows, interleaved by 32-row groups."""
    out = empty_packed(2 * f, k, gate.device) if out is None else out
    check(lib().zest_convert_weight_gu(wtype, _ptr(gate), _ptr(up), f, k, _ptr(out), _stream()),
          "zest_convert_weight_gu")
    return out


def gemm_glu(kind: int, a_packed, m: int, w_gu, f: int, k: int, xout=True, h=None, nonfinite=None):
    """The fused gate/up GEMM: glu(A . gate^T, A . up^T) written as the next
    matmul's expanded operand (xout: True allocates one) and/or fp32 rows h.
    Returns (xout, h)."""
    torch = _torch()
    xo = empty_act(m, f, a_packed.device) if xout is True else xout
    ht = torch.empty((m, f), dtype=torch.float32, device=a_packed.device) if h is True else h
    ldh = ht.stride(0) if ht is not None else 0
    check(lib().zest_gemm_glu(kind, _ptr(a_packed), m, _ptr(w_gu), f, k, _ptr(xo), _ptr(ht), ldh, _ptr(nonfinite),
                              _stream()), "zest_gemm_glu")
    return xo, ht


def rms_norm(x, eps: float, w=None, y=True, packed=None):
    torch = _torch()
    rows, d = x.shape
    yt = torch.empty_like(x) if y is True else y
    check(lib().zest_rms_norm(_ptr(x), rows, d, eps, _ptr(w), _ptr(yt), _ptr(packed), _stream()), "zest_rms_norm")
    return yt


def glu(kind: int, g, u, f: int, sg: int | None = None, su: int | None = None, y=True, packed=None, rows=None):
    torch = _torch()
    rows = g.shape[0] if rows is None else rows
    sg = g.stride(0) if sg is None else sg
    su = u.stride(0) if su is None else su
    yt = torch.empty((rows, f), dtype=torch.float32, device=g.device) if y is True else y
    check(lib().zest_glu(kind, _ptr(g), sg, _ptr(u), su, rows, f, _ptr(yt), _ptr(packed), _stream()), "zest_glu")
    return yt


def add(a, b, b_is_row: bool = False, y=None):
    torch = _torch()
    rows, d = a.shape
    y = torch.empty_like(a) if y is None else y
    check(lib().zest_add(_ptr(a), _ptr(b), rows, d, int(b_is_row), _ptr(y), _stream()), "zest_add")
    return y


def mul_row(x, w, y=None):
    torch = _torch()
    rows, d = x.shape
    y = torch.empty_like(x) if y is None else y
    check(lib().zest_mul_row(_ptr(x), _ptr(w), rows, d, _ptr(y), _stream()), "zest_mul_row")
    return y


def scale(x, s: float, b: float, y=None):
    torch = _torch()
    y = torch.empty_like(x) if y is None else y
    check(lib().zest_scale(_ptr(x), x.numel(), s, b, _ptr(y), _stream()), "zest_scale")
    return y


def check_finite(y, flag):
    """Sets flag[0] (a device uint32/int32 tensor) when y holds NaN or infinity."""
    rows, cols = (y.shape[0], y.shape[1]) if y.dim() == 2 else (1, y.numel())
    ld = y.stride(0) if y.dim() == 2 else cols
    check(lib().zest_check_finite(_ptr(y), rows, cols, ld, _ptr(flag), _stream()), "zest_check_finite")


def rope(x, pos, ff, n_dims: int, mode: int, freq_base: float, freq_scale: float, ext_factor: float,
         attn_factor: float, corr: tuple[float, float], y=None):
    torch = _torch()
    t, heads, d = x.shape
    y = torch.empty_like(x) if y is None else y
    check(lib().zest_rope(_ptr(x), t, heads, d, _ptr(pos), _ptr(ff), n_dims, mode, freq_base, freq_scale, ext_factor,
                          attn_factor, corr[0], corr[1], _ptr(y), _stream()), "zest_rope")
    return y
