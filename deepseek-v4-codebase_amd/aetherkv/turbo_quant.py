"""TurboQuant ("PolarQuant") KV quantiser on MI355X — drop-in for aether_2b/turbo_quant.py.

Same public surface as the reference (aether_2b/turbo_quant.py:49-211):

* ``_wht(x)`` — normalised Walsh-Hadamard transform of the last dim (power of two, else
  ``ValueError``), fp32 result, input never mutated.
* ``PolarQuant(bits, seed=42)`` — ``bits`` in {4, 8} else ``ValueError("bits must be 4 or 8, ...")``;
  ``.encode(x) -> (data, scale)`` with int8 ``[..., D]`` (8-bit) or packed uint8 ``[..., D//2]``
  (4-bit, even element in the low nibble) and fp32 ``[..., 1]`` scale; ``.decode(data, scale,
  out_dtype=torch.bfloat16)``; ``._diag(d, device)`` the cached Rademacher diagonal.

Encode and decode run as single fused HIP kernels (libaetherkv ``aekv_tq_encode`` /
``aekv_tq_decode``) and are bit-exact with the reference's fp32 op sequence.  Tensors must live on
a HIP device; there is no CPU path.
"""
from __future__ import annotations

from typing import Dict, Tuple

import torch

from . import _lib


def _check_pow2(d: int) -> None:
    if d == 0 or (d & (d - 1)) != 0:
        raise ValueError(f"WHT requires last dim to be a power of 2, got {d}")


def _wht(x: torch.Tensor) -> torch.Tensor:
    """Normalised Walsh-Hadamard transform on the last dimension (turbo_quant.py:49-76)."""
    d = x.shape[-1]
    _check_pow2(d)
    _lib.require_device("x", x)
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        x = x.to(torch.float32)
    epl = min(d, 8)
    src = _lib.aligned(x, min(16, epl * x.element_size()))
    out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    n = x.numel() // d
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().aekv_wht(_lib.ptr(src), _lib.dtype_code(src), n, d, _lib.ptr(out), _lib.stream_of(x)),
                   "aekv_wht")
    return out


class PolarQuant:
    """Randomised Hadamard rotation + symmetric absmax scalar quantisation (turbo_quant.py:83-211)."""

    def __init__(self, bits: int, seed: int = 42) -> None:
        if bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {bits}")
        self.bits = bits
        self._seed = seed
        self._diag_cache: Dict[Tuple[int, str], torch.Tensor] = {}

    def _diag(self, d: int, device: torch.device) -> torch.Tensor:
        """Fixed +-1 diagonal for dimension d: MT19937(seed*10007+d) draws, r > 0.5 -> +1."""
        key = (d, str(device))
        if key not in self._diag_cache:
            host = torch.empty(d, dtype=torch.float32)
            _lib.check(_lib.lib().aekv_tq_diag(self._seed, d, _lib.ptr(host)), "aekv_tq_diag")
            self._diag_cache[key] = host.to(device)
        return self._diag_cache[key]

    def encode(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """x [..., D] -> (int8 [..., D] | uint8 [..., D//2], fp32 scale [..., 1])."""
        d = x.shape[-1]
        _check_pow2(d)
        _lib.require_device("x", x)
        if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            x = x.to(torch.float32)
        diag = self._diag(d, x.device)
        epl = min(d, 8)
        src = _lib.aligned(x, min(16, epl * x.element_size()))
        lead = tuple(x.shape[:-1])
        if self.bits == 8:
            data = torch.empty(lead + (d,), dtype=torch.int8, device=x.device)
        else:
            data = torch.empty(lead + (d // 2,), dtype=torch.uint8, device=x.device)
        scale = torch.empty(lead + (1,), dtype=torch.float32, device=x.device)
        n = x.numel() // d
        with torch.cuda.device(x.device):
            _lib.check(_lib.lib().aekv_tq_encode(_lib.ptr(src), _lib.dtype_code(src), n, d, self.bits, _lib.ptr(diag),
                                                 _lib.ptr(data), _lib.ptr(scale), _lib.stream_of(x)),
                       "aekv_tq_encode")
        return data, scale

    def decode(self, data: torch.Tensor, scale: torch.Tensor,
               out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """(codes, scale) -> [..., D] in out_dtype (turbo_quant.py:168-211)."""
        _lib.require_device("data", data, scale)
        want = torch.int8 if self.bits == 8 else torch.uint8
        if data.dtype != want:
            raise RuntimeError(f"{self.bits}-bit PolarQuant codes must be {want}, got {data.dtype}")
        d = data.shape[-1] * (1 if self.bits == 8 else 2)
        _check_pow2(d)
        lead = tuple(data.shape[:-1])
        n = data.numel() // max(data.shape[-1], 1)
        scale_f32 = scale.to(torch.float32).contiguous()
        if scale_f32.numel() != n:
            raise RuntimeError(f"scale must hold one value per vector ({n}), got shape {tuple(scale.shape)}")
        native = out_dtype in (torch.float32, torch.float16, torch.bfloat16)
        odt = out_dtype if native else torch.float32
        out = torch.empty(lead + (d,), dtype=odt, device=data.device)
        epl = min(d, 8)
        codes = _lib.aligned(data, max(1, epl if self.bits == 8 else epl // 2))
        diag = self._diag(d, data.device)
        with torch.cuda.device(data.device):
            _lib.check(_lib.lib().aekv_tq_decode(_lib.ptr(codes), _lib.ptr(scale_f32), n, d, self.bits,
                                                 _lib.ptr(diag), _lib.ptr(out), _lib.dtype_code(out),
                                                 _lib.stream_of(data)),
                       "aekv_tq_decode")
        return out if native else out.to(out_dtype)
