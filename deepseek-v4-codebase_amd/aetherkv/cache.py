"""Quantised KV cache: the engine's state types and quant helpers, and a preallocated code ring.

Drop-in (same names, fields and behaviour as the reference):
  HCAServingState, CSAServingState   aether_2b/serving.py:66-214 (fields, clone, to_dict, from_dict)
  append_seq                         aether_2b/serving.py:32-37 (_append_seq)
  quant_append                       aether_2b/serving.py:327-346 (_quant_append)
  read_compressed, DequantMemo       aether_2b/serving.py:348-376 (_read_compressed and its memo)
  compressed_to_bf16_for_paging      aether_2b/serving.py:378-398
The engine's helpers are methods that read `self._polar_quant`; here the quantiser is an argument.

Block emission (aether_2b/serving.py:495-505 _hca_emit, :557-576 _emit_csa_block): emit_block
pools a block's token entries, applies RoPE and kv_norm and encodes the result in one kernel,
into a CodeRing slot (CodeRing.append_emitted) or into fresh tensors.

CodeRing is the storage the decode path reads instead: codes [B, capacity, D or D/2] and scales
[B, capacity, 1] allocated ahead, a block append encodes straight into the next slots (capacity
doubles when full, so appends are amortised O(1) instead of the O(S) torch.cat of _append_seq),
and the decode kernels read the whole storage with the visible block count passed separately
(csa_decode_ring, hca_decode_ring), so nothing is copied or dequantised per step.
"""
from __future__ import annotations

from dataclasses import dataclass, fields
from typing import Dict, Optional, Tuple

import torch

from . import _lib
from .decode import csa_decode_step, csa_indexer_topk_quant, quant_sink_attention
from .turbo_quant import PolarQuant

_COUNTERS = ("token_count", "loaded_prefix_tokens")


def _clone(x: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if x is None else x.detach().clone()


def _to_cpu(x: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if x is None else x.detach().cpu()


class _ServingState:
    """clone / to_dict / from_dict over the dataclass fields: the two counters are ints, every other
    field an optional tensor (moved to the CPU by to_dict, to `device` by from_dict)."""

    KIND = ""

    def clone(self):
        return type(self)(**{f.name: (getattr(self, f.name) if f.name in _COUNTERS else _clone(getattr(self, f.name)))
                             for f in fields(self)})

    def to_dict(self) -> Dict[str, object]:
        out: Dict[str, object] = {"type": self.KIND}
        for f in fields(self):
            v = getattr(self, f.name)
            out[f.name] = v if f.name in _COUNTERS else _to_cpu(v)
        return out

    @classmethod
    def from_dict(cls, payload: Dict[str, object], device: torch.device):
        kw: Dict[str, object] = {"token_count": int(payload["token_count"]),
                                 "loaded_prefix_tokens": int(payload.get("loaded_prefix_tokens", 0))}
        for f in fields(cls):
            if f.name not in _COUNTERS:
                v = payload.get(f.name)
                kw[f.name] = None if v is None else v.to(device)
        return cls(**kw)


@dataclass
class HCAServingState(_ServingState):
    """Per-layer HCA decode state (aether_2b/serving.py:66-109)."""

    KIND = "hca"
    token_count: int = 0
    loaded_prefix_tokens: int = 0
    compressed: Optional[torch.Tensor] = None
    compressed_scale: Optional[torch.Tensor] = None  # fp32 per block; None: compressed is unquantised
    window: Optional[torch.Tensor] = None
    buffer_c: Optional[torch.Tensor] = None
    buffer_z: Optional[torch.Tensor] = None


@dataclass
class CSAServingState(_ServingState):
    """Per-layer CSA decode state (aether_2b/serving.py:112-214)."""

    KIND = "csa"
    token_count: int = 0
    loaded_prefix_tokens: int = 0
    compressed: Optional[torch.Tensor] = None
    compressed_scale: Optional[torch.Tensor] = None
    index_compressed: Optional[torch.Tensor] = None
    index_compressed_scale: Optional[torch.Tensor] = None
    window: Optional[torch.Tensor] = None
    curr_a_c: Optional[torch.Tensor] = None
    curr_a_z: Optional[torch.Tensor] = None
    curr_b_c: Optional[torch.Tensor] = None
    curr_b_z: Optional[torch.Tensor] = None
    curr_index_a_c: Optional[torch.Tensor] = None
    curr_index_a_z: Optional[torch.Tensor] = None
    curr_index_b_c: Optional[torch.Tensor] = None
    curr_index_b_z: Optional[torch.Tensor] = None
    prev_b_c: Optional[torch.Tensor] = None
    prev_b_z: Optional[torch.Tensor] = None
    prev_index_b_c: Optional[torch.Tensor] = None
    prev_index_b_z: Optional[torch.Tensor] = None


# ---- the engine's quant helpers -------------------------------------------------------------

def append_seq(existing: Optional[torch.Tensor], new_value: torch.Tensor) -> torch.Tensor:
    """[B, D] values become one step [B, 1, D]; appended along dim 1 (a copy of the whole tensor)."""
    step = new_value.unsqueeze(1) if new_value.ndim == 2 else new_value
    return step if existing is None else torch.cat([existing, step], dim=1)


def quant_append(quant: Optional[PolarQuant], existing_data: Optional[torch.Tensor],
                 existing_scale: Optional[torch.Tensor],
                 new_bf16: torch.Tensor) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Encode new block(s) and append codes and scales (quant None: append the bf16 values)."""
    if quant is None:
        return append_seq(existing_data, new_bf16), None
    codes, scale = quant.encode(new_bf16)
    return append_seq(existing_data, codes), append_seq(existing_scale, scale)


class DequantMemo:
    """Decoded caches keyed by (data pointer, data shape, scale pointer, scale shape, dtype); all
    entries are dropped when `limit` is reached (the engine's bounded memo)."""

    def __init__(self, limit: int = 128):
        self.limit = int(limit)
        self._entries: Dict[Tuple, torch.Tensor] = {}

    @staticmethod
    def key(data: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> Tuple:
        return (int(data.data_ptr()), tuple(data.shape), int(scale.data_ptr()), tuple(scale.shape), str(dtype))

    def get(self, key: Tuple) -> Optional[torch.Tensor]:
        return self._entries.get(key)

    def put(self, key: Tuple, value: torch.Tensor) -> None:
        if len(self._entries) >= self.limit:
            self._entries.clear()
        self._entries[key] = value

    def __len__(self) -> int:
        return len(self._entries)


def read_compressed(quant: Optional[PolarQuant], data: Optional[torch.Tensor], scale: Optional[torch.Tensor],
                    out_dtype: torch.dtype, memo: Optional[DequantMemo] = None) -> Optional[torch.Tensor]:
    """data as floating point: decoded when a scale is present (memoised), else returned as is."""
    if data is None:
        return None
    if scale is None or quant is None:
        return data
    key = DequantMemo.key(data, scale, out_dtype)
    if memo is not None:
        hit = memo.get(key)
        if hit is not None:
            return hit
    decoded = quant.decode(data, scale, out_dtype=out_dtype)
    if memo is not None:
        memo.put(key, decoded)
    return decoded


def compressed_to_bf16_for_paging(quant: Optional[PolarQuant], data: Optional[torch.Tensor],
                                  scale: Optional[torch.Tensor], start: int, end: int,
                                  out_dtype: torch.dtype) -> Optional[torch.Tensor]:
    """Blocks [start, end) in out_dtype (None if the cache holds fewer than `end` blocks)."""
    if data is None or data.size(1) < end:
        return None
    part = data[:, start:end]
    if scale is None or quant is None:
        return part
    return quant.decode(part.contiguous(), scale[:, start:end].contiguous(), out_dtype=out_dtype)


# ---- block emission ------------------------------------------------------------------------------

def rope_inv_freq(rope_dim: int, theta: float, device=None) -> torch.Tensor:
    """RoPE frequencies without a config: 1 / theta^(2i / rope_dim) (modeling.py:137-139).  With a
    config (linear / YaRN scaling) pass the model's get_rope_freqs(...)[: rope_dim // 2] instead."""
    freqs = torch.arange(0, rope_dim, 2, dtype=torch.float32)
    return (1.0 / (theta ** (freqs / rope_dim))).to(device)


def block_rope_position(block, m: int, convention: str = "end"):
    """RoPE position of compressed block `block` (int or integer tensor) of m tokens.

    "end" (the default): block·m + m − 1, the block's last token.  This is the position the
    reference uses everywhere but one place: HCA emission in the engine (serving.py:534 passes
    token_count − 1 to _hca_emit, :498) and in the model (modeling.py:285), CSA blocks in the model
    (modeling.py:476-480) and in the engine's batched prefill, which builds its cache with
    _compress_main (serving.py:1146).  At the first query that sees block i (position (i+1)·m) the
    relative RoPE distance is then 1.

    "start": block·m, what the engine's step-by-step CSA emission uses (serving.py:564:
    absolute_token − (m − 1) with absolute_token = token_count − 1, :640).  A cache extended this
    way after a batched prefill mixes the two conventions; pass "start" only to reproduce that
    engine's decode outputs bit for bit."""
    if convention == "end":
        return block * m + (m - 1)
    if convention == "start":
        return block * m
    raise ValueError(f"block_rope_position: convention must be 'end' or 'start', got {convention!r}")


def emit_block(quant: PolarQuant, c: torch.Tensor, z: torch.Tensor, *, bias: Optional[torch.Tensor] = None,
               rope_dim: int = 0, positions=None, inv_freq: Optional[torch.Tensor] = None,
               norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
               out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
               return_vector: bool = False):
    """Pool one block per row and encode it: c, z [B, L, D] bf16 (the buffered kv_proj / z_proj
    entries, z with its slot bias already added as the engine does, or `bias` [L, D] added here);
    RoPE on the last `rope_dim` dims at `positions` [B] (int or tensor); RMSNorm with
    `norm_weight` [D] (kv_norm) and `eps`.  Writes the codes/scales into `out` = (codes [B, ·],
    scale [B, 1]) views (e.g. a ring slot) or fresh tensors [B, 1, ·] / [B, 1, 1].  Returns
    (codes, scale) or (codes, scale, vector [B, D] bf16)."""
    _lib.require_device("c", c, z, bias, norm_weight)
    if c.dtype != torch.bfloat16 or z.dtype != torch.bfloat16 or c.shape != z.shape or c.dim() != 3:
        raise RuntimeError(f"emit_block expects bf16 c, z of one shape [B, L, D], got {c.dtype} {tuple(c.shape)}, "
                           f"{z.dtype} {tuple(z.shape)}")
    B, L, D = c.shape
    dev = c.device
    bits = quant.bits
    rb = D if bits == 8 else D // 2
    cc, zz = c.contiguous(), z.contiguous()
    bb = None if bias is None else bias.to(torch.bfloat16).reshape(L, D).contiguous()
    nw = None if norm_weight is None else norm_weight.to(torch.bfloat16).reshape(D).contiguous()
    pos = None
    inv = None
    if rope_dim:
        if positions is None or inv_freq is None:
            raise RuntimeError("emit_block: rope_dim needs positions and inv_freq")
        pos = torch.as_tensor(positions, dtype=torch.int64, device=dev).reshape(-1).expand(B).contiguous()
        inv = inv_freq.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if out is None:
        codes = torch.empty((B, 1, rb), dtype=torch.int8 if bits == 8 else torch.uint8, device=dev)
        scale = torch.empty((B, 1, 1), dtype=torch.float32, device=dev)
        row_stride = 1
    else:
        codes, scale = out
        row_stride = codes.stride(0) // rb
        if codes.stride(0) != scale.stride(0) * rb or codes.stride(-1) != 1:
            raise RuntimeError("emit_block: out codes/scale must be slots of one [B, n, ·] ring")
    vec = torch.empty((B, D), dtype=torch.bfloat16, device=dev) if return_vector else None
    diag = quant._diag(D, dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().aekv_emit_block(
            _lib.ptr(cc), _lib.ptr(zz), _lib.ptr(bb), B, L, D, int(rope_dim), _lib.ptr(pos), _lib.ptr(inv),
            _lib.ptr(nw), float(eps), bits, _lib.ptr(diag), _lib.ptr(codes), _lib.ptr(scale), row_stride,
            _lib.ptr(vec), _lib.stream_of(c)), "aekv_emit_block")
    return (codes, scale, vec) if return_vector else (codes, scale)


# ---- preallocated code ring -------------------------------------------------------------------

class CodeRing:
    """TurboQuant codes + scales of one cached tensor of a layer, [B, capacity, ·], n blocks valid.

    append() encodes new blocks into slots n.. (capacity doubles when full; the storage is
    zero-filled so slots past n hold finite values); `data`/`scale` are views of the valid blocks,
    `storage` the whole contiguous arrays the decode kernels read with n passed separately.
    """

    def __init__(self, quant: PolarQuant, batch: int, dim: int, *, capacity: int = 256,
                 device: Optional[torch.device] = None):
        if batch < 1 or dim < 1 or capacity < 1:
            raise ValueError(f"CodeRing needs batch, dim, capacity >= 1, got {batch}, {dim}, {capacity}")
        self.quant = quant
        self.batch, self.dim = int(batch), int(dim)
        self.row_bytes = dim if quant.bits == 8 else dim // 2
        self.code_dtype = torch.int8 if quant.bits == 8 else torch.uint8
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.n = 0
        self._codes, self._scale = self._alloc(int(capacity))
        self._visible: Optional[torch.Tensor] = None
        self._all_idx: Optional[torch.Tensor] = None

    def _alloc(self, cap: int) -> Tuple[torch.Tensor, torch.Tensor]:
        return (torch.zeros(self.batch, cap, self.row_bytes, dtype=self.code_dtype, device=self.device),
                torch.zeros(self.batch, cap, 1, dtype=torch.float32, device=self.device))

    @property
    def capacity(self) -> int:
        return self._codes.size(1)

    @property
    def data(self) -> torch.Tensor:
        return self._codes[:, :self.n]

    @property
    def scale(self) -> torch.Tensor:
        return self._scale[:, :self.n]

    @property
    def storage(self) -> Tuple[torch.Tensor, torch.Tensor]:
        return self._codes, self._scale

    def reserve(self, blocks: int) -> None:
        """Make room for `blocks` blocks in total (at least doubling the capacity when it grows)."""
        if blocks <= self.capacity:
            return
        codes, scale = self._alloc(max(int(blocks), 2 * self.capacity))
        codes[:, :self.n].copy_(self._codes[:, :self.n])
        scale[:, :self.n].copy_(self._scale[:, :self.n])
        self._codes, self._scale = codes, scale

    def append(self, new: torch.Tensor) -> None:
        """Encode new blocks [B, D] or [B, m, D] and store them after the valid ones."""
        step = new.unsqueeze(1) if new.dim() == 2 else new
        if step.dim() != 3 or step.size(0) != self.batch or step.size(2) != self.dim:
            raise RuntimeError(f"CodeRing.append expects [{self.batch}, m, {self.dim}], got {tuple(new.shape)}")
        m = step.size(1)
        if m == 0:
            return
        self.reserve(self.n + m)
        codes, scale = self.quant.encode(step)
        self._codes[:, self.n:self.n + m].copy_(codes)
        self._scale[:, self.n:self.n + m].copy_(scale)
        self.n += m
        self._visible = None

    def append_codes(self, codes: torch.Tensor, scale: torch.Tensor) -> None:
        """Store already-encoded blocks (codes [B, m, ·], scales [B, m(, 1)]) after the valid ones,
        e.g. blocks paged back in; nothing is re-encoded."""
        if codes.dim() != 3 or codes.size(0) != self.batch or codes.size(2) != self.row_bytes:
            raise RuntimeError(f"CodeRing.append_codes expects codes [{self.batch}, m, {self.row_bytes}], "
                               f"got {tuple(codes.shape)}")
        m = codes.size(1)
        if scale.numel() != self.batch * m:
            raise RuntimeError(f"CodeRing.append_codes: {scale.numel()} scales for {self.batch} x {m} blocks")
        if m == 0:
            return
        self.reserve(self.n + m)
        self._codes[:, self.n:self.n + m].copy_(codes.view(self.code_dtype))
        self._scale[:, self.n:self.n + m].copy_(scale.reshape(self.batch, m, 1))
        self.n += m
        self._visible = None

    def drop_front(self, m: int) -> None:
        """Remove the first m valid blocks (flushed to pages), keeping the rest in order from slot 0;
        the freed slots are zeroed."""
        m = int(m)
        if m < 0 or m > self.n:
            raise ValueError(f"CodeRing.drop_front({m}) with {self.n} valid blocks")
        if m == 0:
            return
        rest = self.n - m
        if rest:
            self._codes[:, :rest].copy_(self._codes[:, m:self.n].clone())
            self._scale[:, :rest].copy_(self._scale[:, m:self.n].clone())
        self._codes[:, rest:self.n].zero_()
        self._scale[:, rest:self.n].zero_()
        self.n = rest
        self._visible = None

    def append_emitted(self, c: torch.Tensor, z: torch.Tensor, **emit_kwargs) -> None:
        """Pool, RoPE, normalise and encode one block per row (emit_block) straight into slot n."""
        if c.dim() != 3 or c.size(0) != self.batch or c.size(2) != self.dim:
            raise RuntimeError(f"CodeRing.append_emitted expects [{self.batch}, L, {self.dim}], got {tuple(c.shape)}")
        self.reserve(self.n + 1)
        emit_block(self.quant, c, z, out=(self._codes[:, self.n], self._scale[:, self.n]), **emit_kwargs)
        self.n += 1
        self._visible = None

    def visible(self) -> torch.Tensor:
        """int32 [B] filled with n (the indexer's visible block count)."""
        if self._visible is None:
            self._visible = torch.full((self.batch,), self.n, dtype=torch.int32, device=self.device)
        return self._visible

    def all_indices(self) -> torch.Tensor:
        """int64 [B, n] = 0 .. n-1 per row, contiguous (every valid block, for HCA); rebuilt when n
        changes, i.e. per append, not per decode step."""
        if self._all_idx is None or self._all_idx.size(1) != self.n:
            self._all_idx = torch.arange(self.n, dtype=torch.int64, device=self.device).expand(self.batch, self.n).contiguous()
        return self._all_idx

    @classmethod
    def from_tensors(cls, quant: PolarQuant, data: torch.Tensor, scale: torch.Tensor,
                     capacity: Optional[int] = None) -> "CodeRing":
        """A ring holding existing codes [B, n, ·] and scales [B, n(, 1)]."""
        B, n = data.shape[:2]
        dim = data.size(-1) * (1 if quant.bits == 8 else 2)
        ring = cls(quant, B, dim, capacity=max(int(capacity or 0), n, 1), device=data.device)
        ring._codes[:, :n].copy_(data)
        ring._scale[:, :n].copy_(scale.reshape(B, n, 1))
        ring.n = n
        return ring


def csa_decode_ring(q: torch.Tensor, index_q: torch.Tensor, index_weight: torch.Tensor, index_ring: CodeRing,
                    kv_ring: CodeRing, window: Optional[torch.Tensor], sink: torch.Tensor, softmax_scale: float, *,
                    top_k: int = 256, mode: str = "softplus", index_workspace: Optional[torch.Tensor] = None,
                    attention_workspace: Optional[torch.Tensor] = None, out_idx: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """One CSA decode step (aether_2b/serving.py:597-625) over rings: the indexer scans the valid
    index keys, the attention reads the selected blocks and the window.  Returns (out, idx)."""
    if index_ring.n != kv_ring.n:
        raise RuntimeError(f"index ring holds {index_ring.n} blocks, kv ring {kv_ring.n}")
    k = min(int(top_k), kv_ring.n)
    icodes, iscale = index_ring.storage
    codes, scale = kv_ring.storage
    if k > 0 and index_workspace is None and attention_workspace is None and icodes.size(1) == codes.size(1):
        # both rings hold the same capacity: one call, selection and attention fused per row
        return csa_decode_step(q, index_q, index_weight, icodes, iscale, codes, scale, window, sink, softmax_scale, k,
                               kv_quant=kv_ring.quant, index_quant=index_ring.quant, valid=index_ring.visible(),
                               mode=mode, out_idx=out_idx, out=out)
    if k == 0:
        idx = torch.empty((q.size(0), 0), dtype=torch.int64, device=q.device)
    else:
        idx = csa_indexer_topk_quant(index_q, index_weight, icodes, iscale, k, quant=index_ring.quant,
                                     valid=index_ring.visible(), mode=mode, workspace=index_workspace, out=out_idx)
    o = quant_sink_attention(q, codes, scale, idx, window, sink, softmax_scale, quant=kv_ring.quant,
                             workspace=attention_workspace, out=out)
    return o, idx


def hca_decode_ring(q: torch.Tensor, kv_ring: CodeRing, window: Optional[torch.Tensor], sink: torch.Tensor,
                    softmax_scale: float, *, workspace: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One HCA decode step (aether_2b/serving.py:507-522) over a ring: every valid block + window.
    The ring's data / scale views are read in place (the first n blocks of each storage row)."""
    return quant_sink_attention(q, kv_ring.data, kv_ring.scale, None, window, sink, softmax_scale,
                                quant=kv_ring.quant, workspace=workspace, out=out)
