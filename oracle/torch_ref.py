"""The reference's torch op sequences for the compressed-KV path, on the CPU — TEST INFRASTRUCTURE ONLY.

This module is a checker and a timing baseline, never part of the product: only ``tests/`` (which pin
the C oracle's rounding points against it) and ``bench.py``'s ``cpu_baseline`` leg (which times the
reference's own CPU path with it) use it.  It restates, in the torch eager ops the reference writes
(paths relative to the reference repository root):

* ``wht``, ``encode``, ``decode``: ``_wht`` and ``PolarQuant.encode/decode``,
  aether_2b/turbo_quant.py:49-76, :127-166, :168-211;
* ``index_scores``: the CSA indexer, einsum -> relu -> x weight -> sum over heads,
  aether_2b/serving.py:616-619 (weight rule "raw") and aether_2b/modeling.py:609-611 ("softplus");
* ``sink_attention``: PytorchAttentionBackend.sparse_attention, aether_pipeline/serving.py:99-143;
* ``csa_decode_step``: the CSA decode step over quantised caches, aether_2b/serving.py:597-625
  (dequantise the index and KV caches, score, topk, gather, concat the window, attend with K = V).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn.functional as F


def wht(x: torch.Tensor) -> torch.Tensor:
    """turbo_quant.py:49-76: fp32 butterflies h = 1, 2, .., d/2 as [a + b, a - b] per 2h block, then
    times d ** -0.5."""
    d = x.shape[-1]
    if d == 0 or (d & (d - 1)) != 0:
        raise ValueError(f"WHT requires last dim to be a power of 2, got {d}")
    lead = x.shape[:-1]
    out = x.to(torch.float32)
    h = 1
    while h < d:
        blocks = out.view(*lead, d // (2 * h), 2 * h)
        lo, hi = blocks[..., :h], blocks[..., h:]
        out = torch.cat([lo + hi, lo - hi], dim=-1).view(*lead, d)
        h *= 2
    return out * (d ** -0.5)


def encode(x: torch.Tensor, bits: int, diag: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """turbo_quant.py:127-166 -> (int8 codes or uint8 nibble pairs, fp32 scale [..., 1])."""
    rot = wht(x.float() * diag)
    q_max = 127.0 if bits == 8 else 7.0
    max_abs = rot.abs().amax(dim=-1, keepdim=True).clamp_(min=1e-8)
    scale = max_abs / q_max
    q = (rot / max_abs * q_max).round_().clamp_(-q_max, q_max)
    if bits == 8:
        return q.to(torch.int8), scale
    q = q.to(torch.int32)
    return ((q[..., 0::2] & 0x0F) | ((q[..., 1::2] & 0x0F) << 4)).to(torch.uint8), scale


def unpack(data: torch.Tensor, bits: int) -> torch.Tensor:
    """The code values as fp32 (turbo_quant.py:191-201 for 4-bit: low nibble even, high odd, >= 8 -> -16)."""
    if bits == 8:
        return data.to(torch.float32)
    p = data.to(torch.int32)
    lo, hi = p & 0x0F, (p >> 4) & 0x0F
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    q = torch.empty(*data.shape[:-1], data.shape[-1] * 2, dtype=torch.float32)
    q[..., 0::2] = lo.float()
    q[..., 1::2] = hi.float()
    return q


def decode(data: torch.Tensor, scale: torch.Tensor, bits: int, diag: torch.Tensor,
           out_dtype=torch.bfloat16) -> torch.Tensor:
    """turbo_quant.py:168-211: codes * scale, then _wht, then * diag, cast to out_dtype."""
    rot = unpack(data, bits) * scale.to(torch.float32)
    return (wht(rot) * diag).to(out_dtype)


def index_scores(index_q: torch.Tensor, keys: torch.Tensor, weight: torch.Tensor, rule: str = "softplus") -> torch.Tensor:
    """[B, IH, IC] x [B, S, IC] -> [B, S]: sum_h act(w_h) * relu(q_h . k) (serving.py:618-619 with
    act = identity for "raw"; modeling.py:609-611 with act = softplus)."""
    score = torch.einsum("bhc,bsc->bhs", index_q, keys)
    w = F.softplus(weight) if rule == "softplus" else weight
    return (F.relu(score) * w.unsqueeze(-1)).sum(dim=1)


def sink_attention(q: torch.Tensor, kv: torch.Tensor, topk_indices: torch.Tensor, sink: torch.Tensor,
                   softmax_scale: float) -> torch.Tensor:
    """aether_pipeline/serving.py:99-143: q [B, T, H, D], kv [B, S, 2, D], indices [B, T, K], sink [H]."""
    source = kv.unsqueeze(1).expand(-1, q.size(1), -1, -1, -1)
    index = topk_indices[..., None, None].expand(-1, -1, -1, kv.size(-2), kv.size(-1))
    gathered = torch.gather(source, dim=2, index=index)
    keys, values = gathered[:, :, :, 0, :], gathered[:, :, :, 1, :]
    logits = torch.einsum("bthd,btkd->bthk", q, keys) * softmax_scale
    sink_logits = sink.to(logits.dtype).view(1, 1, -1, 1)
    max_all = torch.maximum(logits.max(dim=-1, keepdim=True).values, sink_logits)
    exp_logits = torch.exp(logits - max_all)
    weights = exp_logits / (exp_logits.sum(dim=-1, keepdim=True) + torch.exp(sink_logits - max_all))
    return torch.einsum("bthk,btkd->bthd", weights, values)


def csa_decode_step(q: torch.Tensor, index_q: torch.Tensor, index_w: torch.Tensor, ix_codes: torch.Tensor,
                    ix_scale: torch.Tensor, kv_codes: torch.Tensor, kv_scale: torch.Tensor, window: torch.Tensor,
                    sink: torch.Tensor, bits: int, diag_ix: torch.Tensor, diag_kv: torch.Tensor, top_k: int,
                    rule: str = "softplus", memo: Optional[dict] = None,
                    compute_dtype=torch.bfloat16) -> Tuple[torch.Tensor, torch.Tensor]:
    """aether_2b/serving.py:597-625 on the CPU: q [B, 1, H, D] bf16, index_q [B, IH, IC] fp32, index_w
    [B, IH] fp32, codes/scales as PolarQuant stores them, window [B, W, D] bf16, sink [H].  The
    dequantised caches are fp32 for the index keys and bf16 for the KV blocks (the engine's dtypes);
    `memo` (a dict) keeps them between calls, as the engine's bounded dequant memo does
    (serving.py:361-376).  The attention runs in compute_dtype (the model's bf16 in the engine,
    _run_backend :450-467).  Returns (out [B, 1, H, D] bf16, idx [B, k])."""
    if memo is not None and "keys" in memo:
        keys, blocks = memo["keys"], memo["blocks"]
    else:
        keys = decode(ix_codes, ix_scale, bits, diag_ix, torch.float32)
        blocks = decode(kv_codes, kv_scale, bits, diag_kv, torch.bfloat16)
        if memo is not None:
            memo["keys"], memo["blocks"] = keys, blocks
    score = index_scores(index_q, keys, index_w, rule)
    k = min(top_k, keys.size(1))
    idx = torch.topk(score, k=k, dim=-1).indices
    gather = idx.unsqueeze(-1).expand(-1, -1, blocks.size(-1))
    sources = torch.cat([torch.gather(blocks, dim=1, index=gather), window], dim=1)
    kv = torch.stack([sources, sources], dim=2)  # K = V (serving.py:52-53)
    full = torch.arange(sources.size(1)).view(1, 1, -1).expand(q.size(0), 1, -1)
    cd = compute_dtype
    out = sink_attention(q.to(cd), kv.to(cd), full, sink.to(cd), q.size(-1) ** -0.5)
    return out.to(torch.bfloat16), idx
