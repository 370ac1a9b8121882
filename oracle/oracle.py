"""CPU oracle for the compressed-KV hot path — TEST INFRASTRUCTURE ONLY.

This module is the checker.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it; the product package (``aetherkv``) never does.

It wraps ``liboracle.so`` (``aekv_oracle.c``, built by ``oracle/Makefile`` with gcc and
``-ffp-contract=off``) with numpy-in / numpy-out helpers.  bf16 and fp16 arrays are passed as
``np.uint16`` bit patterns together with a dtype name.  Each function names the reference
file:line it restates (paths relative to the reference repository root).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Optional, Tuple

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

DTYPES = {"f32": 0, "f16": 1, "bf16": 2}
MODES = {"softplus": 0, "raw": 1, "relu_w": 2}

_lib = None


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the committed Makefile (gcc)."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < (HERE / "aekv_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-C", str(HERE), "-B" if force else "liboracle.so"], check=True,
                       stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, I64, I32, F64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
        L.aekvo_diag.argtypes = [I64, I32, P]
        L.aekvo_wht.argtypes = [P, I32, I64, I32, P, I32]
        L.aekvo_encode.argtypes = [P, I32, I64, I32, I32, P, P, P, I32]
        L.aekvo_decode.argtypes = [P, P, I64, I32, I32, P, P, I32, I32]
        L.aekvo_index_scores.argtypes = [P, P, P, P, I64, I64, I32, I32, I32, P, I32]
        L.aekvo_topk.argtypes = [P, P, I64, I64, I32, P, P]
        L.aekvo_sink_attention.argtypes = [P, P, P, P, I64, I64, I64, I64, I64, I64, I64, F64, P, I32]
        L.aekvo_quant_attention.argtypes = [P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I32,
                                            F64, P, I32]
        L.aekvo_hca_compress.argtypes = [P, P, I64, I64, I64, P]
        L.aekvo_emit_block.argtypes = [P, P, P, I64, I64, I64, I32, P, P, P, ctypes.c_float, P]
        L.aekvo_rope_rmsnorm.argtypes = [P, I64, I64, I64, P, I32, P, I32, P, ctypes.c_float, P]
        L.aekvo_wht_scale.argtypes = [I32]
        L.aekvo_wht_scale.restype = ctypes.c_float
        L.aekvo_softplus.argtypes = [F64]
        L.aekvo_softplus.restype = F64
        _lib = L
    return _lib


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---- scalar formats (c10::BFloat16 RNE; IEEE binary16 RNE) -----------------------------------
def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def wht_scale(d: int) -> np.float32:
    """fp32(d ** -0.5) — turbo_quant.py:76."""
    return np.float32(lib().aekvo_wht_scale(d))


# ---- TurboQuant ------------------------------------------------------------------------------
def diag(seed: int, d: int) -> np.ndarray:
    """PolarQuant._diag — turbo_quant.py:111-121 (MT19937, seed*10007+d)."""
    out = np.empty(d, dtype=np.float32)
    lib().aekvo_diag(seed, d, _p(out))
    return out


def wht(x: np.ndarray, x_dtype: str = "f32", threads: int = 0) -> np.ndarray:
    """_wht — turbo_quant.py:49-76.  x: [..., d] float32 (or uint16 bits with x_dtype)."""
    x = _c(x, np.float32 if x_dtype == "f32" else np.uint16)
    d = x.shape[-1]
    out = np.empty(x.shape, dtype=np.float32)
    if lib().aekvo_wht(_p(x), DTYPES[x_dtype], x.size // max(d, 1), d, _p(out), threads) != 0:
        raise ValueError(f"WHT requires last dim to be a power of 2, got {d}")
    return out


def encode(x: np.ndarray, x_dtype: str, bits: int, diag_vec: np.ndarray,
           threads: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """PolarQuant.encode — turbo_quant.py:127-166.  Returns (codes, scale[..., 1])."""
    x = _c(x, np.float32 if x_dtype == "f32" else np.uint16)
    d = x.shape[-1]
    n = x.size // d
    lead = x.shape[:-1]
    codes = np.empty(lead + ((d,) if bits == 8 else (d // 2,)), dtype=np.int8 if bits == 8 else np.uint8)
    scale = np.empty(lead + (1,), dtype=np.float32)
    rc = lib().aekvo_encode(_p(x), DTYPES[x_dtype], n, d, bits, _p(_c(diag_vec, np.float32)),
                            _p(codes), _p(scale), threads)
    if rc != 0:
        raise ValueError("bad encode arguments")
    return codes, scale


def decode(codes: np.ndarray, scale: np.ndarray, bits: int, diag_vec: np.ndarray,
           out_dtype: str = "bf16", threads: int = 0) -> np.ndarray:
    """PolarQuant.decode — turbo_quant.py:168-211.  bf16/f16 results as uint16 bits."""
    codes = _c(codes, np.int8 if bits == 8 else np.uint8)
    d = codes.shape[-1] * (1 if bits == 8 else 2)
    n = codes.size // codes.shape[-1]
    out = np.empty(codes.shape[:-1] + (d,), dtype=np.float32 if out_dtype == "f32" else np.uint16)
    rc = lib().aekvo_decode(_p(codes), _p(_c(scale, np.float32)), n, d, bits,
                            _p(_c(diag_vec, np.float32)), _p(out), DTYPES[out_dtype], threads)
    if rc != 0:
        raise ValueError("bad decode arguments")
    return out


# ---- CSA indexer -----------------------------------------------------------------------------
def index_scores(q: np.ndarray, w: np.ndarray, keys: np.ndarray, valid: Optional[np.ndarray] = None,
                 mode: str = "softplus", threads: int = 0) -> np.ndarray:
    """Indexer scores in double (modeling.py:609-611 / serving.py:618-619 / csa_indexer_cuda.cu:44-55).

    q [B,IH,IC] f32, w [B,IH] f32, keys [B,S,IC] f32 -> [B,S] float64 (-inf beyond valid[b])."""
    q, w, keys = _c(q, np.float32), _c(w, np.float32), _c(keys, np.float32)
    B, IH, IC = q.shape
    S = keys.shape[1]
    out = np.empty((B, S), dtype=np.float64)
    v = None if valid is None else _c(valid, np.int32)
    lib().aekvo_index_scores(_p(q), _p(w), _p(keys), _p(v), B, S, IH, IC, MODES[mode], _p(out), threads)
    return out


def topk(scores: np.ndarray, k: int, valid: Optional[np.ndarray] = None) -> Tuple[np.ndarray, np.ndarray]:
    """Top-k by (score desc, index asc), padded with -1 beyond valid[b]."""
    scores = _c(scores, np.float64)
    B, S = scores.shape
    idx = np.empty((B, k), dtype=np.int64)
    sc = np.empty((B, k), dtype=np.float64)
    v = None if valid is None else _c(valid, np.int32)
    lib().aekvo_topk(_p(scores), _p(v), B, S, k, _p(idx), _p(sc))
    return idx, sc


# ---- attention -------------------------------------------------------------------------------
def sink_attention(q: np.ndarray, kv: np.ndarray, idx: np.ndarray, sink: np.ndarray, scale: float,
                   threads: int = 0) -> np.ndarray:
    """aether_pipeline/serving.py:99-143 with the CUDA kernel's skip of out-of-range indices."""
    q, kv = _c(q, np.float32), _c(kv, np.float32)
    idx, sink = _c(idx, np.int64), _c(np.atleast_1d(sink), np.float32)
    B, T, H, D = q.shape
    S, K = kv.shape[1], idx.shape[2]
    out = np.empty_like(q)
    lib().aekvo_sink_attention(_p(q), _p(kv), _p(idx), _p(sink), sink.size, B, T, H, D, S, K,
                               float(scale), _p(out), threads)
    return out


def quant_attention(q: np.ndarray, codes: np.ndarray, scale: np.ndarray, sel: Optional[np.ndarray],
                    window: np.ndarray, sink: np.ndarray, diag_vec: np.ndarray, bits: int,
                    sm_scale: float, threads: int = 0) -> np.ndarray:
    """Decode-step attention over dequantised (bf16) blocks + bf16 window — serving.py:507-522, :597-625.

    q [B,H,D] f32 (bf16-valued), codes [B,S,*], scale [B,S(,1)], sel [B,K] int64 or None (all S),
    window [B,W,D] f32 (bf16-valued), sink [H] f32."""
    q, window = _c(q, np.float32), _c(window, np.float32)
    codes = _c(codes, np.int8 if bits == 8 else np.uint8)
    scale = _c(scale, np.float32)
    B, H, D = q.shape
    S = codes.shape[1]
    W = window.shape[1]
    K = 0 if sel is None else sel.shape[1]
    s = None if sel is None else _c(sel, np.int64)
    out = np.empty((B, H, D), dtype=np.float32)
    lib().aekvo_quant_attention(_p(q), _p(codes), _p(scale), _p(s), _p(window),
                                _p(_c(sink, np.float32)), _p(_c(diag_vec, np.float32)), B, H, D, S, K,
                                W, bits, float(sm_scale), _p(out), threads)
    return out


def hca_compress(c: np.ndarray, z: np.ndarray) -> np.ndarray:
    """serving.py:495-497 / sparse_attention.py:70-83 — softmax over M, weighted sum (double)."""
    c, z = _c(c, np.float32), _c(z, np.float32)
    B, M, D = c.shape
    out = np.empty((B, D), dtype=np.float32)
    lib().aekvo_hca_compress(_p(c), _p(z), B, M, D, _p(out))
    return out


def emit_block(c: np.ndarray, z: np.ndarray, bias: Optional[np.ndarray] = None, rope_dim: int = 0,
               pos: Optional[np.ndarray] = None, inv_freq: Optional[np.ndarray] = None,
               norm_w: Optional[np.ndarray] = None, eps: float = 1e-6) -> np.ndarray:
    """Block emission (serving.py:495-505, :557-576): bf16 bit patterns (uint16) in and out.
    c, z [B, L, D]; bias [L, D]; pos int64 [B]; inv_freq fp32 [rope_dim/2]; norm_w [D]."""
    c, z = _c(c, np.uint16), _c(z, np.uint16)
    B, L, D = c.shape
    out = np.empty((B, D), dtype=np.uint16)
    bias = None if bias is None else _c(bias, np.uint16)
    pos = None if pos is None else _c(pos, np.int64)
    inv_freq = None if inv_freq is None else _c(inv_freq, np.float32)
    norm_w = None if norm_w is None else _c(norm_w, np.uint16)
    rc = lib().aekvo_emit_block(_p(c), _p(z), _p(bias), B, L, D, int(rope_dim), _p(pos), _p(inv_freq), _p(norm_w),
                                ctypes.c_float(eps), _p(out))
    if rc != 0:
        raise ValueError(f"aekvo_emit_block failed ({rc})")
    return out


def rope_rmsnorm(x: np.ndarray, pos: np.ndarray, inv_freq: Optional[np.ndarray], rope_dim: int,
                 norm_w: Optional[np.ndarray] = None, eps: float = 1e-6, sign: int = 1) -> np.ndarray:
    """serving.py:437-448 / 469-472 — RoPE at sign * pos[row] then optional RMSNorm (bf16 points).

    x [rows, heads, D] uint16 (bf16 bits), pos [rows] int64 -> uint16 [rows, heads, D]."""
    x = _c(x, np.uint16)
    rows, heads, D = x.shape
    out = np.empty_like(x)
    p = _c(np.asarray(pos, dtype=np.int64).reshape(rows), np.int64)
    f = None if inv_freq is None else _c(inv_freq, np.float32)
    w = None if norm_w is None else _c(norm_w, np.uint16)
    rc = lib().aekvo_rope_rmsnorm(_p(x), rows, heads, D, _p(p), int(sign), _p(f), int(rope_dim), _p(w),
                                  ctypes.c_float(eps), _p(out))
    if rc != 0:
        raise ValueError("bad rope_rmsnorm arguments")
    return out


def softplus(x: float) -> float:
    return float(lib().aekvo_softplus(float(x)))
