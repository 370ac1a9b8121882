"""Quantised compressed-KV decode step on MI355X: CSA indexer + top-k + sparse sink attention, and
HCA block attention, reading TurboQuant codes directly (no dequantised cache is materialised).

What the reference decode step does (aether_2b/serving.py):
  CSA  :597-625  dequantise the whole index cache and KV cache (_read_compressed :346-376), score
                 blocks (einsum -> relu -> x weight -> sum over heads, :618-619), topk(min(256, S)),
                 gather, concat the bf16 window, attend with the sink (_run_backend :450-467).
  HCA  :507-522  dequantise every visible block, concat the window, attend with full indices.
Here each step is two fused HIP stages: the indexer scans the index codes in the rotated domain and
selects the top-k exactly; the attention kernel gathers the selected code rows, dequantises them on
load to the same bf16 values PolarQuant.decode produces, and attends them together with the window
and the per-head sink (split over source tiles, merged with the sink counted once).

Score rule: ``mode="softplus"`` (aether_2b/modeling.py:609-611, default), ``"raw"`` (the serving
engine's sum_h w_h relu(q_h.k), serving.py:618-619) or ``"relu_w"`` (csa_indexer_cuda.cu:44-55).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from .turbo_quant import PolarQuant


def _check_out(name: str, t: torch.Tensor, dtype: torch.dtype, numel: int, device) -> None:
    """A caller-supplied output buffer goes to the kernels as a raw pointer: it must have the
    dtype, element count and device the kernels write, and be contiguous."""
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.numel() != numel:
        raise RuntimeError(f"{name} must hold {numel} elements, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if t.device != (device if isinstance(device, torch.device) else torch.device(device)):
        raise RuntimeError(f"{name} must be on {device}, got {t.device}")


# The decode entry points are called once per layer and token, so their host cost counts: a tensor
# conversion or view builds a new tensor object (≈ 0.5–0.7 us each) even when it changes nothing,
# so inputs already in the kernels' form are passed as they are.
def _f32(t: torch.Tensor) -> torch.Tensor:
    """t as contiguous fp32 (t itself when it already is)."""
    if t.dtype != torch.float32:
        t = t.to(torch.float32)
    return t.contiguous()


def _i32(t: torch.Tensor) -> torch.Tensor:
    """t as contiguous int32 (t itself when it already is)."""
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _sink_f32(sink: torch.Tensor, H: int) -> torch.Tensor:
    """The per-head sink as H contiguous fp32 values (a scalar is broadcast)."""
    sk = _f32(sink)
    n = sk.numel()
    if n == 1 and H != 1:
        return sk.reshape(1).expand(H).contiguous()
    if n != H:
        raise RuntimeError("sink must be a scalar or a [num_heads] tensor")
    return sk


def _like_q(out: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    """The output in q's shape (a view only when the caller's buffer has another)."""
    return out if out.dim() == q.dim() else out.view(q.shape)


def _iptr(t: Optional[torch.Tensor]) -> Optional[int]:
    """Device address as a plain int (None stays None), for the entry points called per token."""
    return None if t is None else t.data_ptr()


def _scale_2d(scale: torch.Tensor, B: int, S: int) -> torch.Tensor:
    s = _f32(scale)
    if s.numel() != B * S:
        raise RuntimeError(f"scale must hold B*S = {B * S} values, got shape {tuple(scale.shape)}")
    return s


def _prefix_rows(codes: torch.Tensor, scale: torch.Tensor) -> Optional[int]:
    """Row stride S when codes [B, n, rb] and scale fp32 [B, n] / [B, n, 1] are the first n rows of
    [B, S, ·] storages (a CodeRing's data / scale views): the kernels then read them in place, as
    the first n blocks of rows S apart.  None when they are laid out otherwise."""
    if codes.dim() != 3 or scale.dtype != torch.float32 or scale.dim() not in (2, 3):
        return None
    B, n, rb = codes.shape
    if codes.stride(2) != 1 or codes.stride(1) != rb or codes.stride(0) % rb:
        return None
    S = codes.stride(0) // rb
    if scale.size(0) != B or scale.size(1) != n or (scale.dim() == 3 and scale.size(2) != 1):
        return None
    if scale.stride(0) != S or (n > 1 and scale.stride(1) != 1) or S < n:
        return None
    return S


def indexer_workspace(B: int, S: int, k: int, device) -> torch.Tensor:
    return torch.empty(_lib.lib().aekv_csa_indexer_workspace_size(B, S, k), dtype=torch.uint8, device=device)


def attention_workspace(B: int, H: int, D: int, n_comp: int, W: int, device) -> torch.Tensor:
    return torch.empty(_lib.lib().aekv_quant_attention_workspace_size(B, H, D, n_comp, W), dtype=torch.uint8,
                       device=device)


def csa_indexer_topk_quant(index_q: torch.Tensor, index_weight: torch.Tensor, key_codes: torch.Tensor,
                           key_scale: torch.Tensor, k: int, *, quant: PolarQuant,
                           valid: Optional[torch.Tensor] = None, mode: str = "softplus",
                           return_scores: bool = False, workspace: Optional[torch.Tensor] = None,
                           out: Optional[torch.Tensor] = None):
    """Top-k block indices [B, k] (int64, sorted by score desc then index asc; -1 pads rows whose
    valid count is below k) over TurboQuant-coded index keys.

    index_q [B, IH, IC] fp32, index_weight [B, IH] fp32 (raw; the rule applies softplus),
    key_codes [B, S, IC] int8 (8-bit) or [B, S, IC/2] uint8 (4-bit), key_scale [B, S(, 1)] fp32,
    valid [B] int32 visible block count per row (None: all S).
    """
    _lib.require_device("index_q", index_q, index_weight, key_codes, key_scale, valid)
    if mode not in _lib.INDEX_MODES:
        raise ValueError(f"mode must be one of {sorted(_lib.INDEX_MODES)}, got {mode!r}")
    B, IH, IC = index_q.shape
    S = key_codes.size(1)
    bits = quant.bits
    want = torch.int8 if bits == 8 else torch.uint8
    if key_codes.dtype != want:
        raise RuntimeError(f"{bits}-bit index codes must be {want}, got {key_codes.dtype}")
    if key_codes.size(-1) * (1 if bits == 8 else 2) != IC or key_codes.size(0) != B:
        raise RuntimeError(f"key_codes shape {tuple(key_codes.shape)} does not match index_q {tuple(index_q.shape)}")
    q = index_q.to(torch.float32).contiguous()
    w = index_weight.to(torch.float32).contiguous()
    codes = key_codes.contiguous()
    sc = _scale_2d(key_scale, B, S)
    v = None if valid is None else valid.to(torch.int32).contiguous()
    diag = quant._diag(IC, index_q.device)
    L = _lib.lib()
    if out is None:
        out = torch.empty((B, k), dtype=torch.int64, device=index_q.device)
    else:
        _check_out("out", out, torch.int64, B * k, index_q.device)
    scores = torch.empty((B, k), dtype=torch.float32, device=index_q.device) if return_scores else None
    if workspace is None:
        workspace = indexer_workspace(B, S, k, index_q.device)
    with torch.cuda.device(index_q.device):
        _lib.check(L.aekv_csa_indexer_topk_quant(
            _lib.ptr(q), _lib.ptr(w), _lib.ptr(codes), _lib.ptr(sc), _lib.ptr(diag), _lib.ptr(v), B, S, IH, IC, bits,
            int(k), _lib.INDEX_MODES[mode], _lib.ptr(workspace), workspace.numel(), _lib.ptr(out), _lib.ptr(scores),
            _lib.stream_of(index_q)), "aekv_csa_indexer_topk_quant")
    return (out, scores) if return_scores else out


def quant_sink_attention(q: torch.Tensor, codes: torch.Tensor, scale: torch.Tensor, sel: Optional[torch.Tensor],
                         window: Optional[torch.Tensor], sink: torch.Tensor, softmax_scale: float, *,
                         quant: PolarQuant, workspace: Optional[torch.Tensor] = None,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode-step sink attention over [dequant(codes[sel]) ; window] with K = V.

    q [B, 1, H, D] or [B, H, D] bf16; codes [B, S, D] int8 | [B, S, D/2] uint8; scale [B, S(, 1)];
    sel [B, K] int64 block indices (None: all S blocks — HCA); window [B, W, D] bf16 or None;
    sink [H].  Returns bf16 with q's shape.
    """
    _lib.require_device("q", q, codes, scale, sel, window, sink)
    if q.dtype != torch.bfloat16:
        raise RuntimeError(f"q must be bfloat16, got {q.dtype}")
    qs = q.shape
    if len(qs) == 4 and qs[1] != 1:
        raise RuntimeError("quant_sink_attention expects one target token per row")
    if len(qs) not in (3, 4):
        raise RuntimeError(f"q must be [B, 1, H, D] or [B, H, D], got {tuple(qs)}")
    B, H, D = qs[0], qs[-2], qs[-1]
    S = codes.size(1)
    bits = quant.bits
    want = torch.int8 if bits == 8 else torch.uint8
    if codes.dtype != want:
        raise RuntimeError(f"{bits}-bit codes must be {want}, got {codes.dtype}")
    if codes.size(-1) * (1 if bits == 8 else 2) != D or codes.size(0) != B:
        raise RuntimeError(f"codes shape {tuple(codes.shape)} does not match q {tuple(q.shape)}")
    qc = q.contiguous()
    s64 = None if sel is None else (sel if sel.dtype == torch.int64 else sel.to(torch.int64)).contiguous()
    K = -1 if s64 is None else s64.size(1)  # n_sel < 0: every block (HCA)
    stride = _prefix_rows(codes, scale) if s64 is None and not codes.is_contiguous() else None
    if stride is not None:
        # every block of row prefixes (e.g. a ring's valid blocks): read in place, rows `stride` apart
        cc, sc, K = codes, scale, S
    else:
        cc, sc = codes.contiguous(), _scale_2d(scale, B, S)
    if window is not None and window.numel() > 0:
        if window.dtype != torch.bfloat16 or window.dim() != 3 or window.size(0) != B or window.size(2) != D:
            raise RuntimeError(f"window must be bf16 [B, W, D], got {window.dtype} {tuple(window.shape)}")
        win = window.contiguous()
        W = win.size(1)
    else:
        win, W = None, 0
    sk = _sink_f32(sink, H)
    diag = quant._diag(D, q.device)
    n_comp = K if K >= 0 else S
    if workspace is None:
        workspace = attention_workspace(B, H, D, n_comp, W, q.device)
    dev = q.device
    if out is None:
        out = torch.empty(qs, dtype=torch.bfloat16, device=dev)
    else:
        _check_out("out", out, torch.bfloat16, B * H * D, dev)
    with _lib.on_device(dev):
        rc = _lib.hot("aekv_quant_sink_attention")(
            qc.data_ptr(), cc.data_ptr(), sc.data_ptr(), _iptr(s64), _iptr(win), sk.data_ptr(), diag.data_ptr(), B, H,
            D, S if stride is None else stride, K, W, bits, float(softmax_scale), workspace.data_ptr(),
            workspace.numel(), out.data_ptr(), _lib.raw_stream(dev))
    _lib.check(rc, "aekv_quant_sink_attention")
    return _like_q(out, q)


def decode_workspace(B: int, S: int, k: int, H: int, D: int, W: int, device) -> torch.Tensor:
    """Workspace of csa_decode_step (the indexer's and the attention's)."""
    return torch.empty(_lib.lib().aekv_csa_decode_workspace_size(B, S, k, H, D, W), dtype=torch.uint8, device=device)


def csa_decode_step(q: torch.Tensor, index_q: torch.Tensor, index_weight: torch.Tensor, index_codes: torch.Tensor,
                    index_scale: torch.Tensor, kv_codes: torch.Tensor, kv_scale: torch.Tensor,
                    window: Optional[torch.Tensor], sink: torch.Tensor, softmax_scale: float, k: int, *,
                    kv_quant: PolarQuant, index_quant: PolarQuant, valid: Optional[torch.Tensor] = None,
                    mode: str = "softplus", return_scores: bool = False, workspace: Optional[torch.Tensor] = None,
                    out_idx: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    """The CSA decode step in one call (aekv_csa_decode_quant): the indexer's top-k of the visible
    index keys, then the sink attention over those blocks and the window.  Same results as
    csa_indexer_topk_quant followed by quant_sink_attention; the per-row selection and attention run
    in one kernel where the matrix-core kernels apply.  Index codes [B, S, IC(/2)] and KV codes
    [B, S, D(/2)] cover the same S blocks.  Returns (out like q, idx [B, k]) or, with return_scores,
    (out, idx, scores [B, k])."""
    _lib.require_device("q", q, index_q, index_weight, index_codes, index_scale, kv_codes, kv_scale, window, sink,
                        valid)
    if mode not in _lib.INDEX_MODES:
        raise ValueError(f"mode must be one of {sorted(_lib.INDEX_MODES)}, got {mode!r}")
    if q.dtype != torch.bfloat16:
        raise RuntimeError(f"q must be bfloat16, got {q.dtype}")
    qs = q.shape
    if len(qs) == 4 and qs[1] != 1:
        raise RuntimeError("csa_decode_step expects one target token per row")
    if len(qs) not in (3, 4):
        raise RuntimeError(f"q must be [B, 1, H, D] or [B, H, D], got {tuple(qs)}")
    q3 = q.contiguous()
    B, H, D = qs[0], qs[-2], qs[-1]
    IB, IH, IC = index_q.shape
    S = kv_codes.size(1)
    if index_codes.size(1) != S or IB != B:
        raise RuntimeError(f"index codes {tuple(index_codes.shape)} and KV codes {tuple(kv_codes.shape)} must cover "
                           f"the same B rows and S blocks")
    for name, quant, codes, dim in (("index", index_quant, index_codes, IC), ("KV", kv_quant, kv_codes, D)):
        want = torch.int8 if quant.bits == 8 else torch.uint8
        if codes.dtype != want:
            raise RuntimeError(f"{quant.bits}-bit {name} codes must be {want}, got {codes.dtype}")
        if codes.size(-1) * (1 if quant.bits == 8 else 2) != dim or codes.size(0) != B:
            raise RuntimeError(f"{name} codes shape {tuple(codes.shape)} does not match head dim {dim} and batch {B}")
    if window is not None and window.numel() > 0:
        if window.dtype != torch.bfloat16 or window.dim() != 3 or window.size(0) != B or window.size(2) != D:
            raise RuntimeError(f"window must be bf16 [B, W, D], got {window.dtype} {tuple(window.shape)}")
        win = _lib.aligned(window, 16)
        W = win.size(1)
    else:
        win, W = None, 0
    sk = _sink_f32(sink, H)
    iq = _f32(index_q)
    iw = _f32(index_weight)
    ic = index_codes.contiguous()
    isc = _scale_2d(index_scale, B, S)
    kc = _lib.aligned(kv_codes, 16)
    ksc = _scale_2d(kv_scale, B, S)
    v = None if valid is None else _i32(valid)
    dev = q.device
    idiag = index_quant._diag(IC, dev)
    kdiag = kv_quant._diag(D, dev)
    L = _lib.lib()
    if out_idx is None:
        out_idx = torch.empty((B, k), dtype=torch.int64, device=dev)
    else:
        _check_out("out_idx", out_idx, torch.int64, B * k, dev)
    scores = torch.empty((B, k), dtype=torch.float32, device=dev) if return_scores else None
    if out is None:
        out = torch.empty(qs, dtype=torch.bfloat16, device=dev)
    else:
        _check_out("out", out, torch.bfloat16, B * H * D, dev)
    if workspace is None:
        workspace = decode_workspace(B, S, k, H, D, W, dev)
    with _lib.on_device(dev):
        rc = _lib.hot("aekv_csa_decode_quant")(
            iq.data_ptr(), iw.data_ptr(), ic.data_ptr(), isc.data_ptr(), idiag.data_ptr(), _iptr(v), B, S, IH, IC,
            index_quant.bits, int(k), _lib.INDEX_MODES[mode], q3.data_ptr(), kc.data_ptr(), ksc.data_ptr(), _iptr(win),
            sk.data_ptr(), kdiag.data_ptr(), H, D, W, kv_quant.bits, float(softmax_scale), workspace.data_ptr(),
            workspace.numel(), out_idx.data_ptr(), _iptr(scores), out.data_ptr(), _lib.raw_stream(dev))
    _lib.check(rc, "aekv_csa_decode_quant")
    o = _like_q(out, q)
    return (o, out_idx, scores) if return_scores else (o, out_idx)


def csa_decode(q: torch.Tensor, index_q: torch.Tensor, index_weight: torch.Tensor, index_codes: torch.Tensor,
               index_scale: torch.Tensor, kv_codes: torch.Tensor, kv_scale: torch.Tensor,
               window: Optional[torch.Tensor], sink: torch.Tensor, softmax_scale: float, *, kv_quant: PolarQuant,
               index_quant: Optional[PolarQuant] = None, top_k: int = 256, mode: str = "softplus",
               valid: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """One CSA decode step (serving.py:597-625): returns (attention output like q, selected [B, k])."""
    index_quant = index_quant or kv_quant
    S = kv_codes.size(1)
    k = min(int(top_k), S)
    if k == 0:
        return quant_sink_attention(q, kv_codes, kv_scale, kv_codes.new_zeros((q.size(0), 0), dtype=torch.int64),
                                    window, sink, softmax_scale, quant=kv_quant), None
    return csa_decode_step(q, index_q, index_weight, index_codes, index_scale, kv_codes, kv_scale, window, sink,
                           softmax_scale, k, kv_quant=kv_quant, index_quant=index_quant, valid=valid, mode=mode)


def hca_decode(q: torch.Tensor, kv_codes: torch.Tensor, kv_scale: torch.Tensor, window: Optional[torch.Tensor],
               sink: torch.Tensor, softmax_scale: float, *, kv_quant: PolarQuant) -> torch.Tensor:
    """One HCA decode step (serving.py:507-522): all blocks + window."""
    return quant_sink_attention(q, kv_codes, kv_scale, None, window, sink, softmax_scale, quant=kv_quant)
