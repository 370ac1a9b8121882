"""Kernel entry points with the reference signatures — drop-in for aether_kernels/sparse_attention.py.

Reference: aether_kernels/sparse_attention.py:8-83 (wrappers) and aether_kernels/csrc/bindings.cpp
(argument checks, same messages, raised as RuntimeError like TORCH_CHECK).

* ``sparse_sink_attention(q, kv, topk_indices, sink, softmax_scale)``
* ``tiled_prefill_attention(q, kv, sink, softmax_scale, tile_size=256)``
* ``csa_indexer_topk(index_q, index_kv, index_weight, k, *, mode="relu_w")``
* ``hca_compress(buffer_c, buffer_z)``

Outputs are freshly allocated tensors on the inputs' device; kernels run on the current stream.  The
attention calls also take a split workspace from torch's caching allocator when the matrix-core
launch would leave most CUs idle (few targets, many sources).
"""
from __future__ import annotations

import torch

from . import _lib


def _check_input(name: str, t: torch.Tensor) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _check_sink(sink: torch.Tensor, heads: int) -> None:
    if not (sink.numel() == 1 or (sink.dim() == 1 and sink.size(0) == heads)):
        raise RuntimeError("sink must be a scalar or a [num_heads] tensor")


def _workspace(nbytes: int, device):
    """Split workspace for the matrix-core attention (torch's caching allocator; None: no split)."""
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes > 0 else None


def _ext_sparse_sink_attention(q, kv, topk_indices, sink, softmax_scale):
    """bindings.cpp:21-46 checks, then aekv_sparse_sink_attention."""
    for n, t in (("q", q), ("kv", kv), ("topk_indices", topk_indices), ("sink", sink)):
        _check_input(n, t)
    if q.dim() != 4:
        raise RuntimeError("q must have shape [B, T, H, D]")
    if kv.dim() != 4:
        raise RuntimeError("kv must have shape [B, S, 2, D]")
    if kv.size(2) != 2:
        raise RuntimeError("kv third dimension must be 2 for [K, V]")
    if topk_indices.dim() != 3:
        raise RuntimeError("topk_indices must have shape [B, T, K]")
    if q.size(0) != kv.size(0):
        raise RuntimeError("q and kv batch dimensions must match")
    if q.size(0) != topk_indices.size(0):
        raise RuntimeError("q and topk_indices batch dimensions must match")
    if q.size(1) != topk_indices.size(1):
        raise RuntimeError("q and topk_indices target-token dimensions must match")
    if q.size(3) != kv.size(3):
        raise RuntimeError("q and kv head dimensions must match")
    if topk_indices.dtype not in (torch.int64, torch.int32):
        raise RuntimeError("topk_indices must be int32 or int64")
    _check_sink(sink, q.size(2))
    if kv.dtype != q.dtype or sink.dtype != q.dtype:
        raise RuntimeError("q, kv and sink must share one floating dtype")
    B, T, H, D = q.shape
    out = torch.empty_like(q)
    L = _lib.lib()
    K = topk_indices.size(2)
    ws = _workspace(L.aekv_sink_attention_workspace_size(_lib.dtype_code(q), B, T, H, D, kv.size(1), K), q.device)
    with torch.cuda.device(q.device):
        _lib.check(L.aekv_sparse_sink_attention_ws(
            _lib.ptr(q), _lib.ptr(kv), _lib.ptr(topk_indices), _lib.dtype_code(topk_indices), _lib.ptr(sink),
            sink.numel(), _lib.dtype_code(q), B, T, H, D, kv.size(1), K, float(softmax_scale),
            _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.ptr(out), _lib.stream_of(q)),
            "aekv_sparse_sink_attention")
    return out


def _ext_tiled_prefill_attention(q, kv, sink, softmax_scale, tile_size):
    """bindings.cpp:58-77 checks, then aekv_tiled_prefill_attention (sink counted once)."""
    for n, t in (("q", q), ("kv", kv), ("sink", sink)):
        _check_input(n, t)
    if q.dim() != 4:
        raise RuntimeError("q must have shape [B, T, H, D]")
    if kv.dim() != 4:
        raise RuntimeError("kv must have shape [B, S, 2, D]")
    if kv.size(2) != 2:
        raise RuntimeError("kv third dimension must be 2 for [K, V]")
    if q.size(0) != kv.size(0):
        raise RuntimeError("q and kv batch dimensions must match")
    if q.size(3) != kv.size(3):
        raise RuntimeError("q and kv head dimensions must match")
    if tile_size <= 0:
        raise RuntimeError("tile_size must be positive")
    _check_sink(sink, q.size(2))
    if kv.dtype != q.dtype or sink.dtype != q.dtype:
        raise RuntimeError("q, kv and sink must share one floating dtype")
    B, T, H, D = q.shape
    out = torch.empty_like(q)
    L = _lib.lib()
    ws = _workspace(L.aekv_sink_attention_workspace_size(_lib.dtype_code(q), B, T, H, D, kv.size(1), -1), q.device)
    with torch.cuda.device(q.device):
        _lib.check(L.aekv_tiled_prefill_attention_ws(
            _lib.ptr(q), _lib.ptr(kv), _lib.ptr(sink), sink.numel(), _lib.dtype_code(q), B, T, H, D, kv.size(1),
            float(softmax_scale), int(tile_size), _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.ptr(out),
            _lib.stream_of(q)), "aekv_tiled_prefill_attention")
    return out


def _ext_csa_indexer_topk(index_q, index_kv, index_weight, k, mode="relu_w"):
    """bindings.cpp:88-101 and csa_indexer_cuda.cu:88-95 checks, then aekv_csa_indexer_topk."""
    for n, t in (("index_q", index_q), ("index_kv", index_kv), ("index_weight", index_weight)):
        _check_input(n, t)
    if index_q.dim() != 3:
        raise RuntimeError("index_q must have shape [B, IH, IC]")
    if index_kv.dim() != 3:
        raise RuntimeError("index_kv must have shape [B, S, IC]")
    if index_weight.dim() != 2:
        raise RuntimeError("index_weight must have shape [B, IH]")
    if k <= 0:
        raise RuntimeError("k must be positive")
    for n, t in (("index_q", index_q), ("index_kv", index_kv), ("index_weight", index_weight)):
        if t.dtype != torch.float32:
            raise RuntimeError(f"{n} must be float32")
    B, IH, IC = index_q.shape
    S = index_kv.size(1)
    if not (0 < k <= S):
        raise RuntimeError("k must be in [1, S]")
    if index_kv.size(0) != B or index_kv.size(2) != IC or tuple(index_weight.shape) != (B, IH):
        raise RuntimeError("index_q, index_kv and index_weight shapes do not match")
    if mode not in _lib.INDEX_MODES:
        raise ValueError(f"mode must be one of {sorted(_lib.INDEX_MODES)}, got {mode!r}")
    L = _lib.lib()
    out = torch.empty((B, k), dtype=torch.int64, device=index_q.device)
    ws = torch.empty(L.aekv_csa_indexer_workspace_size(B, S, k), dtype=torch.uint8, device=index_q.device)
    with torch.cuda.device(index_q.device):
        _lib.check(L.aekv_csa_indexer_topk(
            _lib.ptr(index_q), _lib.ptr(index_kv), _lib.ptr(index_weight), None, B, S, IH, IC, int(k),
            _lib.INDEX_MODES[mode], _lib.ptr(ws), ws.numel(), _lib.ptr(out), None, _lib.stream_of(index_q)),
            "aekv_csa_indexer_topk")
    return out


def _ext_hca_compress(buffer_c, buffer_z):
    """bindings.cpp:110-119 checks, then aekv_hca_compress."""
    _check_input("buffer_c", buffer_c)
    _check_input("buffer_z", buffer_z)
    if buffer_c.dim() != 3:
        raise RuntimeError("buffer_c must have shape [B, M, D]")
    if buffer_z.dim() != 3:
        raise RuntimeError("buffer_z must have shape [B, M, D]")
    if buffer_c.shape != buffer_z.shape:
        raise RuntimeError("buffer_c and buffer_z must have the same shape")
    if buffer_z.dtype != buffer_c.dtype:
        raise RuntimeError("buffer_c and buffer_z must share one floating dtype")
    B, M, D = buffer_c.shape
    out = torch.empty((B, D), dtype=buffer_c.dtype, device=buffer_c.device)
    with torch.cuda.device(buffer_c.device):
        _lib.check(_lib.lib().aekv_hca_compress(_lib.ptr(buffer_c), _lib.ptr(buffer_z), _lib.dtype_code(buffer_c), B, M,
                                                D, _lib.ptr(out), _lib.stream_of(buffer_c)), "aekv_hca_compress")
    return out


# ---- public wrappers (sparse_attention.py:8-83) ----------------------------------------------
def sparse_sink_attention(q: torch.Tensor, kv: torch.Tensor, topk_indices: torch.Tensor, sink: torch.Tensor,
                          softmax_scale: float) -> torch.Tensor:
    return _ext_sparse_sink_attention(q, kv, topk_indices, sink, float(softmax_scale))


def tiled_prefill_attention(q: torch.Tensor, kv: torch.Tensor, sink: torch.Tensor, softmax_scale: float,
                            tile_size: int = 256) -> torch.Tensor:
    """Sink attention of every target over all S sources; the sink enters the normaliser once
    (aether_2b/modeling.py:158-178 semantics)."""
    return _ext_tiled_prefill_attention(q.contiguous(), kv.contiguous(), sink.contiguous(), float(softmax_scale),
                                        int(tile_size))


def csa_indexer_topk(index_q: torch.Tensor, index_kv: torch.Tensor, index_weight: torch.Tensor, k: int, *,
                     mode: str = "relu_w") -> torch.Tensor:
    """Fused indexer score + top-k -> [B, k] int64, sorted by (score desc, index asc).

    The default is the rule of the reference function this replaces, so an unchanged caller gets
    the same selection (up to fp32 near-ties; torch.topk's order among equal scores is unspecified):
    mode "relu_w":   sum_h max(w_h,0) (q_h.k)         (aether_kernels/csrc/csa_indexer_cuda.cu:44-55,
                                                       docstring aether_kernels/sparse_attention.py:57)
    The model's and the serving engine's rules are selectable:
    mode "softplus": sum_h softplus(w_h) relu(q_h.k)  (aether_2b/modeling.py:609-611)
    mode "raw":      sum_h w_h relu(q_h.k)            (aether_2b/serving.py:618-619)
    """
    return _ext_csa_indexer_topk(index_q.float().contiguous(), index_kv.float().contiguous(),
                                 index_weight.float().contiguous(), int(k), mode)


def hca_compress(buffer_c: torch.Tensor, buffer_z: torch.Tensor) -> torch.Tensor:
    """Softmax over the M window positions of buffer_z, weighted sum of buffer_c -> [B, D]."""
    return _ext_hca_compress(buffer_c.contiguous(), buffer_z.contiguous())
