"""Query-side and output-side work around the attention step on MI355X.

What the reference does per attention call (aether_2b/serving.py):
  _query         :437-442  q = q_norm(apply_rope(q_up(q_down(x)), position))
  _window_entry  :444-448  entry = kv_norm(apply_rope(window_kv(x), position))
  _post_attention :469-472 y = output(apply_rope(out, -position)) with the grouped output projection
                           (modeling.py:187-203: heads in output_groups groups, one Linear per group,
                           concatenated, then out_proj)
Each apply_rope + RMSNorm is ~12 separate bf16 torch ops (slices, cos/sin, repeat_interleave, two
products, a stack for the rotation, a cat, the norm).  Here each is one launch of
aekv_rope_rmsnorm (one wave per head vector, same rounding points); the projections stay library
GEMMs (torch.nn.functional.linear on the device, i.e. hipBLASLt), fed by the rotated output.
"""
from __future__ import annotations

from typing import Optional, Sequence, Union

import torch
import torch.nn.functional as F

from . import _lib

Positions = Union[int, torch.Tensor]


def _row_positions(positions: Positions, lead: Sequence[int], device) -> torch.Tensor:
    """int64 [rows] for a tensor with leading dims `lead` (rows = prod(lead)): an int, a [T] tensor
    (the last leading dim, shared by the batch as the reference's 1-D positions) or a tensor of
    shape `lead`."""
    rows = 1
    for n in lead:
        rows *= int(n)
    if isinstance(positions, int):
        return torch.full((rows,), positions, dtype=torch.int64, device=device)
    p = positions.to(device=device, dtype=torch.int64)
    if p.dim() == 0:
        return p.expand(rows).contiguous()
    if p.dim() == 1 and len(lead) >= 1 and p.numel() == int(lead[-1]):
        return p.expand(*lead).reshape(rows).contiguous()
    if tuple(p.shape) == tuple(int(n) for n in lead):
        return p.reshape(rows).contiguous()
    raise RuntimeError(f"positions of shape {tuple(p.shape)} do not match leading dims {tuple(lead)}")


def rope_rmsnorm(x: torch.Tensor, positions: Positions, *, rope_dim: int, inv_freq: Optional[torch.Tensor],
                 norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6, inverse: bool = False,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """apply_rope on the last rope_dim dims at each row's position (negated when `inverse`), then
    RMSNorm with norm_weight when given.  x [..., heads, D] bf16 with D = 128 or 256; positions as
    for the leading dims x.shape[:-2]; inv_freq fp32 [rope_dim / 2] (get_rope_freqs or
    cache.rope_inv_freq).  Returns a tensor like x (or writes `out`, which may be x)."""
    _lib.require_device("x", x)
    if x.dtype != torch.bfloat16 or x.dim() < 2:
        raise RuntimeError(f"x must be bfloat16 [..., heads, D], got {x.dtype} {tuple(x.shape)}")
    heads, D = int(x.size(-2)), int(x.size(-1))
    lead = tuple(x.shape[:-2]) or (1,)
    rows = 1
    for n in lead:
        rows *= int(n)
    xc = _lib.aligned(x, 8)
    pos = _row_positions(positions, lead, x.device) if rope_dim > 0 else None
    f = None
    if rope_dim > 0:
        if inv_freq is None:
            raise ValueError("rope_dim > 0 needs inv_freq")
        f = inv_freq.to(device=x.device, dtype=torch.float32).contiguous()
        if f.numel() < rope_dim // 2:
            raise RuntimeError(f"inv_freq has {f.numel()} entries, rope_dim {rope_dim} needs {rope_dim // 2}")
    w = None
    if norm_weight is not None:
        w = norm_weight.to(device=x.device, dtype=torch.bfloat16).contiguous()
        if w.numel() != D:
            raise RuntimeError(f"norm_weight has {w.numel()} entries, expected {D}")
    if out is None:
        out = torch.empty_like(xc)
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().aekv_rope_rmsnorm(
            _lib.ptr(xc), rows, heads, D, _lib.ptr(pos), -1 if inverse else 1, _lib.ptr(f), int(rope_dim), _lib.ptr(w),
            float(eps), _lib.ptr(out), _lib.stream_of(x)), "aekv_rope_rmsnorm")
    return out


def query_prep(q: torch.Tensor, positions: Positions, inv_freq: torch.Tensor, *, rope_dim: int,
               q_norm_weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """q_norm(apply_rope(q, positions)) for q [B, T, H, D] (or [B, H, D]) bf16 — serving.py:437-442."""
    return rope_rmsnorm(q, positions, rope_dim=rope_dim, inv_freq=inv_freq, norm_weight=q_norm_weight, eps=eps)


def window_entry(kv: torch.Tensor, positions: Positions, inv_freq: torch.Tensor, *, rope_dim: int,
                 kv_norm_weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """kv_norm(apply_rope(kv, positions)) for window entries kv [B, T, D] bf16 — serving.py:444-448."""
    y = rope_rmsnorm(kv.unsqueeze(-2), positions, rope_dim=rope_dim, inv_freq=inv_freq, norm_weight=kv_norm_weight,
                     eps=eps)
    return y.squeeze(-2)


def grouped_output_projection(x: torch.Tensor, group_weights: Sequence[torch.Tensor],
                              out_proj_weight: torch.Tensor) -> torch.Tensor:
    """GroupedOutputProjection.forward (modeling.py:187-203) for x [..., H, D]: the heads split into
    len(group_weights) groups, group g flattened and multiplied by group_weights[g]
    [group_out, H/G * D], the results concatenated and multiplied by out_proj_weight
    [hidden, G * group_out] (no biases)."""
    G = len(group_weights)
    if G == 0 or x.size(-2) % G:
        raise RuntimeError(f"{x.size(-2)} heads do not split into {G} groups")
    chunks = x.chunk(G, dim=-2)
    projected = [F.linear(c.flatten(-2), w) for c, w in zip(chunks, group_weights)]
    return F.linear(torch.cat(projected, dim=-1), out_proj_weight)


def post_attention(out: torch.Tensor, positions: Positions, inv_freq: torch.Tensor, *, rope_dim: int,
                   group_weights: Sequence[torch.Tensor], out_proj_weight: torch.Tensor) -> torch.Tensor:
    """attn.output(apply_rope(out, -positions)) for out [B, H, D] or [B, T, H, D] — serving.py:469-472,
    modeling.py:326-337 (per target).  Returns [B, hidden] or [B, T, hidden]."""
    rotated = rope_rmsnorm(out, positions, rope_dim=rope_dim, inv_freq=inv_freq, inverse=True)
    return grouped_output_projection(rotated, group_weights, out_proj_weight)
