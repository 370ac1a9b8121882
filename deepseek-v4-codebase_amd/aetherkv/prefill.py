"""Chunked prefill attention through the quantised reader on MI355X.

What the reference does (aether_2b/modeling.py, the ``_forward_tiled_prefill`` paths):
  HCA  :293-337  for every target t: g = min(nb, t // M) compressed blocks, the sliding-window entries
                 [max(0, t - W + 1), t], one tiled_prefill_attention call (sparse_attention.py:19-42)
                 over cat([comp[:, :g], window]) with K = V and the per-head sink.
  CSA  :496-550  the same, but the blocks are the indexer's top-min(K, g) of the first g blocks
                 (softplus-weighted relu scores, :524-530).
Both loop over targets in Python, one kernel launch (and one torch.cat / stack) per token, over the
bf16 compressed blocks.  Here the blocks stay TurboQuant codes: one indexer launch scores every
target of the chunk (each against its own visible prefix), and one attention launch covers every
(target, head) row, gathering and dequantising the code rows on load; each target reads its own
slice of one window buffer.  The positional bookkeeping (which blocks and window entries a target
sees) follows the reference exactly and is computed on the host (:316-320, :521-534).

Not covered here: the query-side projections and the inverse RoPE / output projection around the
attention call (:326-337, :540-550) — callers keep those.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from .decode import _scale_2d
from .turbo_quant import PolarQuant


def prefill_sources(n_targets: int, start: int, n_blocks: int, *, compression: int, sliding_window: int,
                    window_base: int, window_len: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-target source counts of a chunk of targets at positions start .. start + n_targets - 1.

    Returns int32 CPU tensors [n_targets]: visible blocks g = min(n_blocks, p // compression)
    (modeling.py:316/521), and the window slice [max(0, p - W + 1), p] (modeling.py:318-319/532-533)
    as (start, length) relative to a window buffer whose entry i holds position window_base + i and
    which holds window_len entries.  Raises ValueError if the buffer does not cover a slice.
    """
    if n_targets < 0 or start < 0 or n_blocks < 0:
        raise ValueError("n_targets, start and n_blocks must be non-negative")
    if compression < 1 or sliding_window < 1:
        raise ValueError("compression and sliding_window must be positive")
    p = torch.arange(start, start + n_targets, dtype=torch.int64)
    vis = torch.clamp(p // compression, max=n_blocks)
    w_first = torch.clamp(p - sliding_window + 1, min=0)
    ws = w_first - window_base
    wl = p - w_first + 1
    if n_targets and (int(ws.min()) < 0 or int((ws + wl).max()) > window_len):
        raise ValueError(f"window buffer of {window_len} entries from position {window_base} does not cover the "
                         f"sliding windows of positions {start} .. {start + n_targets - 1}")
    return vis.to(torch.int32), ws.to(torch.int32), wl.to(torch.int32)


def prefill_workspace(B: int, T: int, H: int, n_comp: int, Wt: int, device) -> torch.Tensor:
    return torch.empty(_lib.lib().aekv_quant_prefill_workspace_size(B, T, H, n_comp, Wt), dtype=torch.uint8,
                       device=device)


def _rows_i32(x: Optional[torch.Tensor], B: int, T: int, name: str, device) -> Optional[torch.Tensor]:
    if x is None:
        return None
    x = x.to(device=device, dtype=torch.int32)
    if x.dim() == 1:
        x = x.expand(B, T)
    if tuple(x.shape) != (B, T):
        raise RuntimeError(f"{name} must be [T] or [B, T] = [{B}, {T}], got {tuple(x.shape)}")
    return x.contiguous()


def csa_prefill_indexer_topk_quant(index_q: torch.Tensor, index_weight: torch.Tensor, key_codes: torch.Tensor,
                                   key_scale: torch.Tensor, k: int, *, quant: PolarQuant,
                                   valid: Optional[torch.Tensor] = None, mode: str = "softplus",
                                   return_scores: bool = False, workspace: Optional[torch.Tensor] = None,
                                   out: Optional[torch.Tensor] = None):
    """Top-k block indices [B, T, k] for every target of a chunk (modeling.py:524-530).

    index_q [B, T, IH, IC] fp32, index_weight [B, T, IH] fp32, key_codes [B, S, IC or IC/2],
    key_scale [B, S(, 1)], valid [T] or [B, T] int32, host or device: target t scores blocks
    j < valid[b, t] (None: all S).  Rows are sorted by score desc, index asc, and padded with -1.
    """
    _lib.require_device("index_q", index_q, index_weight, key_codes, key_scale)
    if mode not in _lib.INDEX_MODES:
        raise ValueError(f"mode must be one of {sorted(_lib.INDEX_MODES)}, got {mode!r}")
    if index_q.dim() != 4:
        raise RuntimeError(f"index_q must be [B, T, IH, IC], got {tuple(index_q.shape)}")
    B, T, IH, IC = index_q.shape
    S = key_codes.size(1)
    bits = quant.bits
    want = torch.int8 if bits == 8 else torch.uint8
    if key_codes.dtype != want:
        raise RuntimeError(f"{bits}-bit index codes must be {want}, got {key_codes.dtype}")
    if key_codes.size(-1) * (1 if bits == 8 else 2) != IC or key_codes.size(0) != B:
        raise RuntimeError(f"key_codes shape {tuple(key_codes.shape)} does not match index_q {tuple(index_q.shape)}")
    if tuple(index_weight.shape) != (B, T, IH):
        raise RuntimeError(f"index_weight must be [B, T, IH] = [{B}, {T}, {IH}], got {tuple(index_weight.shape)}")
    q = index_q.to(torch.float32).contiguous()
    w = index_weight.to(torch.float32).contiguous()
    codes = key_codes.contiguous()
    sc = _scale_2d(key_scale, B, S)
    v = _rows_i32(valid, B, T, "valid", index_q.device)
    diag = quant._diag(IC, index_q.device)
    L = _lib.lib()
    if out is None:
        out = torch.empty((B, T, k), dtype=torch.int64, device=index_q.device)
    scores = torch.empty((B, T, k), dtype=torch.float32, device=index_q.device) if return_scores else None
    if workspace is None:
        workspace = torch.empty(L.aekv_csa_indexer_workspace_size(B * T, S, k), dtype=torch.uint8,
                                device=index_q.device)
    with torch.cuda.device(index_q.device):
        _lib.check(L.aekv_csa_prefill_indexer_topk_quant(
            _lib.ptr(q), _lib.ptr(w), _lib.ptr(codes), _lib.ptr(sc), _lib.ptr(diag), _lib.ptr(v), B, T, S, IH, IC,
            bits, int(k), _lib.INDEX_MODES[mode], _lib.ptr(workspace), workspace.numel(), _lib.ptr(out),
            _lib.ptr(scores), _lib.stream_of(index_q)), "aekv_csa_prefill_indexer_topk_quant")
    return (out, scores) if return_scores else out


def quant_prefill_attention(q: torch.Tensor, codes: torch.Tensor, scale: torch.Tensor, sel: Optional[torch.Tensor],
                            window: Optional[torch.Tensor], sink: torch.Tensor, softmax_scale: float, *,
                            quant: PolarQuant, visible: Optional[torch.Tensor] = None,
                            win_start: Optional[torch.Tensor] = None, win_len: Optional[torch.Tensor] = None,
                            workspace: Optional[torch.Tensor] = None,
                            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Sink attention of every target of a chunk over its own quantised blocks and window slice.

    q [B, T, H, 128] bf16 (H <= 16); codes [B, S, D] int8 | [B, S, D/2] uint8; scale [B, S(, 1)];
    sel [B, T, K] int64 block indices (target t uses sel[b, t, :visible[b, t]]; entries outside
    [0, S) skipped) or None (blocks 0 .. visible[b, t]-1 in order — HCA); window [B, Wt, D] bf16;
    visible / win_start / win_len [T] or [B, T] int32, host or device (None: K or S / 0 / the rest of
    the window); sink [H] or scalar.  Returns [B, T, H, D] bf16.
    """
    _lib.require_device("q", q, codes, scale, sel, window, sink)
    if q.dtype != torch.bfloat16 or q.dim() != 4:
        raise RuntimeError(f"q must be bfloat16 [B, T, H, D], got {q.dtype} {tuple(q.shape)}")
    B, T, H, D = q.shape
    S = codes.size(1)
    bits = quant.bits
    want = torch.int8 if bits == 8 else torch.uint8
    if codes.dtype != want:
        raise RuntimeError(f"{bits}-bit codes must be {want}, got {codes.dtype}")
    if codes.size(-1) * (1 if bits == 8 else 2) != D or codes.size(0) != B:
        raise RuntimeError(f"codes shape {tuple(codes.shape)} does not match q {tuple(q.shape)}")
    qc = _lib.aligned(q, 16)
    cc = _lib.aligned(codes, 16)
    sc = _scale_2d(scale, B, S)
    if sel is not None:
        if sel.dim() != 3 or sel.size(0) != B or sel.size(1) != T:
            raise RuntimeError(f"sel must be [B, T, K] = [{B}, {T}, K], got {tuple(sel.shape)}")
        s64 = sel.to(torch.int64).contiguous()
        K = s64.size(2)
    else:
        s64, K = None, -1
    if window is not None and window.numel() > 0:
        if window.dtype != torch.bfloat16 or window.dim() != 3 or window.size(0) != B or window.size(2) != D:
            raise RuntimeError(f"window must be bf16 [B, Wt, D], got {window.dtype} {tuple(window.shape)}")
        win = _lib.aligned(window, 16)
        Wt = win.size(1)
    else:
        win, Wt = None, 0
    sk = sink.to(torch.float32).reshape(-1).contiguous()
    if sk.numel() == 1:
        sk = sk.expand(H).contiguous()
    if sk.numel() != H:
        raise RuntimeError("sink must be a scalar or a [num_heads] tensor")
    vis = _rows_i32(visible, B, T, "visible", q.device)
    ws_ = _rows_i32(win_start, B, T, "win_start", q.device)
    wl = _rows_i32(win_len, B, T, "win_len", q.device)
    diag = quant._diag(D, q.device)
    n_comp = K if K >= 0 else S
    if workspace is None:
        workspace = prefill_workspace(B, T, H, n_comp, Wt, q.device)
    if out is None:
        out = torch.empty((B, T, H, D), dtype=torch.bfloat16, device=q.device)
    with torch.cuda.device(q.device):
        _lib.check(_lib.lib().aekv_quant_prefill_attention(
            _lib.ptr(qc), _lib.ptr(cc), _lib.ptr(sc), _lib.ptr(s64), _lib.ptr(vis), _lib.ptr(win), _lib.ptr(ws_),
            _lib.ptr(wl), _lib.ptr(sk), _lib.ptr(diag), B, T, H, D, S, K, Wt, bits, float(softmax_scale),
            _lib.ptr(workspace), workspace.numel(), _lib.ptr(out), _lib.stream_of(q)), "aekv_quant_prefill_attention")
    return out


def _window_rows(window: torch.Tensor, T: int, start: int, n_blocks: int, compression: int, sliding_window: int,
                 window_base: Optional[int]):
    Wt = window.size(1)
    base = start + T - Wt if window_base is None else int(window_base)
    vis, ws, wl = prefill_sources(T, start, n_blocks, compression=compression, sliding_window=sliding_window,
                                  window_base=base, window_len=Wt)
    return vis, ws, wl


def hca_prefill(q: torch.Tensor, kv_codes: torch.Tensor, kv_scale: torch.Tensor, window: torch.Tensor,
                sink: torch.Tensor, softmax_scale: float, *, kv_quant: PolarQuant, start: int = 0,
                n_blocks: Optional[int] = None, compression: int = 128, sliding_window: int = 128,
                window_base: Optional[int] = None) -> torch.Tensor:
    """HCA attention of a chunk of targets at positions start .. start + T - 1 (modeling.py:293-325).

    q [B, T, H, 128] bf16; kv_codes / kv_scale: the compressed blocks (the first n_blocks valid,
    default all S); window [B, Wt, 128] bf16 whose entry i is position window_base + i (default: it
    ends at the chunk's last target).  Returns the per-target attention [B, T, H, 128] bf16, before
    the reference's inverse RoPE and output projection.
    """
    B, T = q.shape[:2]
    nb = kv_codes.size(1) if n_blocks is None else int(n_blocks)
    vis, ws, wl = _window_rows(window, T, start, nb, compression, sliding_window, window_base)
    dev = q.device
    return quant_prefill_attention(q, kv_codes, kv_scale, None, window, sink, softmax_scale, quant=kv_quant,
                                   visible=vis.to(dev), win_start=ws.to(dev), win_len=wl.to(dev))


def csa_prefill(q: torch.Tensor, index_q: torch.Tensor, index_weight: torch.Tensor, index_codes: torch.Tensor,
                index_scale: torch.Tensor, kv_codes: torch.Tensor, kv_scale: torch.Tensor, window: torch.Tensor,
                sink: torch.Tensor, softmax_scale: float, *, kv_quant: PolarQuant,
                index_quant: Optional[PolarQuant] = None, start: int = 0, n_blocks: Optional[int] = None,
                compression: int = 4, sliding_window: int = 128, top_k: int = 256, mode: str = "softplus",
                window_base: Optional[int] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """CSA attention of a chunk of targets (modeling.py:496-539): per target, the top-min(K, g) of its
    g visible blocks by the indexer, plus its window slice.

    index_q [B, T, IH, IC] fp32, index_weight [B, T, IH] fp32 (raw; softplus applied), index and KV
    codes over the same blocks (the first n_blocks valid).  Returns (out [B, T, H, 128] bf16,
    selected [B, T, min(top_k, n_blocks)] int64 padded with -1, or None when no block exists).
    """
    index_quant = index_quant or kv_quant
    B, T = q.shape[:2]
    nb = kv_codes.size(1) if n_blocks is None else int(n_blocks)
    k_cfg = min(int(top_k), nb) if nb > 0 else 0  # modeling.py:511
    vis, ws, wl = _window_rows(window, T, start, nb, compression, sliding_window, window_base)
    dev = q.device
    if k_cfg == 0:
        idx = None
        sel = torch.zeros((B, T, 0), dtype=torch.int64, device=dev)
        n_sel = torch.zeros_like(vis)
    else:
        idx = csa_prefill_indexer_topk_quant(index_q, index_weight, index_codes, index_scale, k_cfg,
                                             quant=index_quant, valid=vis.to(dev), mode=mode)
        sel = idx
        n_sel = torch.clamp(vis, max=k_cfg)  # k_eff = min(K, g), modeling.py:527
    out = quant_prefill_attention(q, kv_codes, kv_scale, sel, window, sink, softmax_scale, quant=kv_quant,
                                  visible=n_sel.to(dev), win_start=ws.to(dev), win_len=wl.to(dev))
    return out, idx
