"""Shared test plumbing: the package loader, the CPU oracle and the reference
packer (oracle/_ref) through ctypes, and numpy wrappers around them."""
from __future__ import annotations

import ctypes
import importlib.util
import os
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
sys.path.insert(0, str(GOLDEN))


def load_pkg():
    """The ggml-xdna_amd package, imported as ggml_xdna_amd."""
    if "ggml_xdna_amd" in sys.modules:
        return sys.modules["ggml_xdna_amd"]
    spec = importlib.util.spec_from_file_location(
        "ggml_xdna_amd", ROOT / "ggml-xdna_amd" / "__init__.py",
        submodule_search_locations=[str(ROOT / "ggml-xdna_amd")])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ggml_xdna_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def load_quant():
    load_pkg()
    import ggml_xdna_amd.quant as q  # noqa: E402
    return q


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class Oracle:
    """ctypes over oracle/liboracle.so (strict build) or liboracle_fast.so."""

    def __init__(self, fast: bool = False):
        path = ROOT / "oracle" / ("liboracle_fast.so" if fast else "liboracle.so")
        if not path.exists():
            raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
        L = self.L = ctypes.CDLL(str(path))
        sig = {
            "orc_bfp16_encode_rows": [_P, _I64, _I64, _P],
            "orc_bfp16_decode_rows": [_P, _I64, _I64, _P],
            "orc_pack_a": [_P, _I64, _I64, _I, _I, _P],
            "orc_pack_b": [_P, _I64, _I64, _I, _I, _I, _P],
            "orc_dequant_row": [_I, _P, _P, _I64],
            "orc_ref_mul_mat": [_I, _P, _I64, _I64, _P, _I64, _P, _I],
            "orc_ref_mul_mat_f32": [_P, _I64, _I64, _P, _I64, _P, _I],
            "orc_mul_mat_f64": [_P, _I64, _I64, _P, _I64, _P, _P, _I],
            "orc_rms_norm": [_P, _I64, _I64, _F, _P],
            "orc_mul_row": [_P, _I64, _I64, _P, _P],
            "orc_add": [_P, _P, _I64, _P],
            "orc_add_row": [_P, _I64, _I64, _P, _P],
            "orc_scale": [_P, _I64, _F, _F, _P],
            "orc_glu": [_I, _P, _I64, _P, _I64, _I64, _I64, _P],
            "orc_rope_yarn_corr_dims": [_I, _I, _F, _F, _F, _P],
            "orc_rope": [_P, _I64, _I64, _I64, _P, _P, _I, _I, _I, _F, _F, _F, _F, _F, _F, _P],
            "orc_self_test_inputs": [_I64, _I64, _I64, _P, _P],
        }
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes, f.restype = args, None
        L.orc_a_offset.argtypes, L.orc_a_offset.restype = [_I64, _I64, _I64, _I, _I], ctypes.c_size_t
        L.orc_b_offset.argtypes, L.orc_b_offset.restype = [_I64, _I64, _I64, _I64, _I, _I, _I], ctypes.c_size_t
        L.orc_row_bytes.argtypes, L.orc_row_bytes.restype = [_I, _I64], ctypes.c_size_t
        L.orc_quantize_row.argtypes, L.orc_quantize_row.restype = [_I, _P, _P, _I64], ctypes.c_int

    def encode_rows(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, k = x.reshape(-1, x.shape[-1]).shape
        out = np.empty((rows, k // 8, 9), dtype=np.uint8)
        self.L.orc_bfp16_encode_rows(_ptr(x), rows, k, _ptr(out))
        return out

    def decode_rows(self, b: np.ndarray) -> np.ndarray:
        b = np.ascontiguousarray(b, dtype=np.uint8)
        rows, nb = b.shape[0], b.shape[1]
        out = np.empty((rows, nb * 8), dtype=np.float32)
        self.L.orc_bfp16_decode_rows(_ptr(b), rows, nb * 8, _ptr(out))
        return out

    def pack_a(self, x: np.ndarray, m: int, k: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.size // 8 * 9, dtype=np.uint8)
        self.L.orc_pack_a(_ptr(x), x.shape[0], x.shape[1], m, k, _ptr(out))
        return out

    def pack_b(self, w: np.ndarray, n: int, k: int, cols: int) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty(w.size // 8 * 9, dtype=np.uint8)
        self.L.orc_pack_b(_ptr(w), w.shape[0], w.shape[1], n, k, cols, _ptr(out))
        return out

    def dequant(self, wtype: int, raw: np.ndarray, n: int, k: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        rb = self.L.orc_row_bytes(wtype, k)
        out = np.empty((n, k), dtype=np.float32)
        for r in range(n):
            self.L.orc_dequant_row(wtype, ctypes.c_void_p(raw.ctypes.data + r * rb), ctypes.c_void_p(out.ctypes.data + r * k * 4), k)
        return out

    def row_bytes(self, wtype: int, k: int) -> int:
        return int(self.L.orc_row_bytes(wtype, k))

    def quantize(self, wtype: int, w: np.ndarray) -> np.ndarray:
        """Synthetic GGUF rows of `wtype` from float rows w[n][k]."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        n, k = w.shape
        rb = self.row_bytes(wtype, k)
        out = np.empty((n, rb), dtype=np.uint8)
        for r in range(n):
            st = self.L.orc_quantize_row(wtype, ctypes.c_void_p(w.ctypes.data + r * k * 4),
                                         ctypes.c_void_p(out.ctypes.data + r * rb), k)
            if st != 0:
                raise ValueError(f"no quantiser for type {wtype} at k={k}")
        return out

    def ref_mul_mat(self, wtype: int, raw: np.ndarray, n: int, k: int, x: np.ndarray, threads: int = 8) -> np.ndarray:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty((x.shape[0], n), dtype=np.float32)
        self.L.orc_ref_mul_mat(wtype, _ptr(raw), n, k, _ptr(x), x.shape[0], _ptr(y), threads)
        return y

    def mul_mat_f32(self, w: np.ndarray, x: np.ndarray, threads: int = 8) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty((x.shape[0], w.shape[0]), dtype=np.float32)
        self.L.orc_ref_mul_mat_f32(_ptr(w), w.shape[0], w.shape[1], _ptr(x), x.shape[0], _ptr(y), threads)
        return y

    def mul_mat_f64(self, w: np.ndarray, x: np.ndarray, threads: int = 8):
        w = np.ascontiguousarray(w, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty((x.shape[0], w.shape[0]), dtype=np.float64)
        ab = np.empty_like(y)
        self.L.orc_mul_mat_f64(_ptr(w), w.shape[0], w.shape[1], _ptr(x), x.shape[0], _ptr(y), _ptr(ab), threads)
        return y, ab

    def rms_norm(self, x, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        self.L.orc_rms_norm(_ptr(x), x.shape[0], x.shape[1], eps, _ptr(y))
        return y

    def mul_row(self, x, w):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        y = np.empty_like(x)
        self.L.orc_mul_row(_ptr(x), x.shape[0], x.shape[1], _ptr(w), _ptr(y))
        return y

    def add(self, a, b):
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        y = np.empty_like(a)
        self.L.orc_add(_ptr(a), _ptr(b), a.size, _ptr(y))
        return y

    def add_row(self, x, w):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        y = np.empty_like(x)
        self.L.orc_add_row(_ptr(x), x.shape[0], x.shape[1], _ptr(w), _ptr(y))
        return y

    def scale(self, x, s, b):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        self.L.orc_scale(_ptr(x), x.size, s, b, _ptr(y))
        return y

    def glu(self, kind, g, u):
        g = np.ascontiguousarray(g, dtype=np.float32)
        u = np.ascontiguousarray(u, dtype=np.float32)
        rows, f = g.shape
        y = np.empty((rows, f), dtype=np.float32)
        self.L.orc_glu(kind, _ptr(g), f, _ptr(u), f, rows, f, _ptr(y))
        return y

    def corr_dims(self, n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow):
        d = np.zeros(2, dtype=np.float32)
        self.L.orc_rope_yarn_corr_dims(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, _ptr(d))
        return float(d[0]), float(d[1])

    def rope(self, x, pos, ff, n_dims, mode, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor,
             beta_fast, beta_slow):
        x = np.ascontiguousarray(x, dtype=np.float32)
        pos = np.ascontiguousarray(pos, dtype=np.int32)
        ff = None if ff is None else np.ascontiguousarray(ff, dtype=np.float32)
        y = np.empty_like(x)
        t, h, d = x.shape
        self.L.orc_rope(_ptr(x), t, h, d, _ptr(pos), _ptr(ff), n_dims, mode, n_ctx_orig, freq_base, freq_scale,
                        ext_factor, attn_factor, beta_fast, beta_slow, _ptr(y))
        return y

    def self_test_inputs(self, m, k, n):
        a = np.empty((m, k), dtype=np.float32)
        w = np.empty((n, k), dtype=np.float32)
        self.L.orc_self_test_inputs(m, k, n, _ptr(a), _ptr(w))
        return a, w


class RefPacker:
    """ctypes over the reference's own packer, built from its source into
    oracle/_ref (exists only where the reference tree was present at build)."""

    def __init__(self, flavour: str = "avx2"):
        path = ROOT / "oracle" / "_ref" / f"libbfp16_ref_{flavour}.so"
        if not path.exists():
            raise FileNotFoundError(path)
        L = self.L = ctypes.CDLL(str(path))
        L.ref_encode_block.argtypes = [_P, _P]
        L.ref_pack_a.argtypes = [_P, _I64, _I64, _I, _I, _P]
        L.ref_pack_b.argtypes = [_P, _I64, _I64, _I, _I, _I, _P]
        L.ref_a_offset.argtypes, L.ref_a_offset.restype = [_I64, _I64, _I64, _I, _I], ctypes.c_size_t
        L.ref_b_offset.argtypes, L.ref_b_offset.restype = [_I64, _I64, _I64, _I64, _I, _I, _I], ctypes.c_size_t

    def encode_blocks(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 8)
        out = np.empty((x.shape[0], 9), dtype=np.uint8)
        for i in range(x.shape[0]):
            self.L.ref_encode_block(ctypes.c_void_p(x.ctypes.data + i * 32), ctypes.c_void_p(out.ctypes.data + i * 9))
        return out

    def pack_a(self, x, m, k):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.size // 8 * 9, dtype=np.uint8)
        self.L.ref_pack_a(_ptr(x), x.shape[0], x.shape[1], m, k, _ptr(out))
        return out

    def pack_b(self, w, n, k, cols):
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty(w.size // 8 * 9, dtype=np.uint8)
        self.L.ref_pack_b(_ptr(w), w.shape[0], w.shape[1], n, k, cols, _ptr(out))
        return out


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def nrmse(got: np.ndarray, want: np.ndarray) -> float:
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    return float(np.sqrt(((got - want) ** 2).sum() / max((want ** 2).sum(), 1e-300)))


def gemm_check(g: np.ndarray, r64: np.ndarray, absdot: np.ndarray, k: int, rel: float = 0.0):
    """The GEMM bar: |g - r64| <= rel*|r64| + 2*K*2^-24*sum_k|a_k b_k| for
    every output. The bf16 x bf16 products are exact in fp32, so the only
    difference from the fp64 sum is fp32 summation order, which any order
    keeps inside the second term (K roundings of at most 2^-24 relative each,
    doubled for slack); rel = 0 leaves no room for a systematic error. Also
    returns the max relative error over outputs not near zero (the north
    star's tolerance is 1e-3)."""
    g = g.astype(np.float64)
    err = np.abs(g - r64)
    bound = rel * np.abs(r64) + 2.0 * k * 2.0 ** -24 * absdot
    worst = float((err / np.maximum(bound, 1e-300)).max())
    rms = float(np.sqrt((r64 ** 2).mean()))
    big = np.abs(r64) >= 1e-2 * rms
    maxrel = float((err[big] / np.abs(r64[big])).max()) if big.any() else 0.0
    return worst, maxrel
