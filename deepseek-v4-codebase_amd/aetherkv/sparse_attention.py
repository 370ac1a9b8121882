"""Kernel entry points with the reference signatures — drop-in for aether_kernels/sparse_attention.py.

Reference: aether_kernels/sparse_attention.py:8-83 (wrappers) and aether_kernels/csrc/bindings.cpp
(argument checks, same messages, raised as RuntimeError like TORCH_CHECK).

* ``sparse_sink_attention(q, kv, topk_indices, sink, softmax_scale)``
* ``tiled_prefill_attention(q, kv, sink, softmax_scale, tile_size=256)``
* ``csa_indexer_topk(index_q, index_kv, index_weight, k, *, mode="relu_w")``
* ``hca_compress(buffer_c, buffer_z)``

Outputs are freshly allocated tensors on the inputs' device; kernels run on the current stream.  The
attention calls also take a split workspace when the matrix-core launch would leave most CUs idle
(few targets, many sources): one buffer per (device, stream), reused by the calls on that stream.
The host-side cost per call is kept small because the reference's callers make one call per target
token (modeling.py:322,534): pointers go to the library as plain integers, the stream handle is read
without building a Stream object, the device is switched only when it is not already current, and
workspace sizes are memoised per shape.
"""
from __future__ import annotations

import functools

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


@functools.lru_cache(maxsize=256)
def _ws_bytes(dt: int, B: int, T: int, H: int, D: int, S: int, K: int) -> int:
    return int(_lib.lib().aekv_sink_attention_workspace_size(dt, B, T, H, D, S, K))


_IDX_DTYPES = (torch.int64, torch.int32)


def _sparse_ok(q, kv, topk_indices, sink) -> bool:
    """Every check of _sparse_checks passes (one expression: the checks' cost counts per call)."""
    qs, ks, ts = q.shape, kv.shape, topk_indices.shape
    return (q.is_cuda and kv.is_cuda and topk_indices.is_cuda and sink.is_cuda and q.is_contiguous()
            and kv.is_contiguous() and topk_indices.is_contiguous() and sink.is_contiguous() and len(qs) == 4
            and len(ks) == 4 and ks[2] == 2 and len(ts) == 3 and qs[0] == ks[0] == ts[0] and qs[1] == ts[1]
            and qs[3] == ks[3] and topk_indices.dtype in _IDX_DTYPES
            and (sink.numel() == 1 or (sink.dim() == 1 and sink.size(0) == qs[2])) and kv.dtype == q.dtype
            and sink.dtype == q.dtype)


def _ext_sparse_sink_attention(q, kv, topk_indices, sink, softmax_scale):
    """bindings.cpp:21-46 checks, then aekv_sparse_sink_attention."""
    if not _sparse_ok(q, kv, topk_indices, sink):
        _sparse_checks(q, kv, topk_indices, sink)
    B, T, H, D = q.shape
    S, K = kv.size(1), topk_indices.size(2)
    out = torch.empty_like(q)
    dev = q.device
    dt = _lib.TORCH_TO_AEKV.get(q.dtype)
    if dt is None:
        raise RuntimeError(f"unsupported dtype {q.dtype}")
    st = _lib.raw_stream(dev)
    ws = _lib.workspace(_ws_bytes(dt, B, T, H, D, S, K), dev, st)
    with _lib.on_device(dev):
        rc = _lib.hot("aekv_sparse_sink_attention_ws")(
            q.data_ptr(), kv.data_ptr(), topk_indices.data_ptr(), _lib.I64 if topk_indices.dtype == torch.int64
            else _lib.I32, sink.data_ptr(), sink.numel(), dt, B, T, H, D, S, K, float(softmax_scale),
            None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), out.data_ptr(), st)
    _lib.check(rc, "aekv_sparse_sink_attention")
    return out


def _sparse_checks(q, kv, topk_indices, sink) -> None:
    """The reference's checks in its order, each with its message (raises on the first failure)."""
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


def _tiled_ok(q, kv, sink, tile_size) -> bool:
    """Every check of _tiled_checks passes."""
    qs, ks = q.shape, kv.shape
    return (q.is_cuda and kv.is_cuda and sink.is_cuda and q.is_contiguous() and kv.is_contiguous()
            and sink.is_contiguous() and len(qs) == 4 and len(ks) == 4 and ks[2] == 2 and qs[0] == ks[0]
            and qs[3] == ks[3] and tile_size > 0 and (sink.numel() == 1 or (sink.dim() == 1 and sink.size(0) == qs[2]))
            and kv.dtype == q.dtype and sink.dtype == q.dtype)


def _ext_tiled_prefill_attention(q, kv, sink, softmax_scale, tile_size):
    """bindings.cpp:58-77 checks, then aekv_tiled_prefill_attention (sink counted once)."""
    if not _tiled_ok(q, kv, sink, tile_size):
        _tiled_checks(q, kv, sink, tile_size)
    B, T, H, D = q.shape
    S = kv.size(1)
    out = torch.empty_like(q)
    dev = q.device
    dt = _lib.TORCH_TO_AEKV.get(q.dtype)
    if dt is None:
        raise RuntimeError(f"unsupported dtype {q.dtype}")
    st = _lib.raw_stream(dev)
    ws = _lib.workspace(_ws_bytes(dt, B, T, H, D, S, -1), dev, st)
    with _lib.on_device(dev):
        rc = _lib.hot("aekv_tiled_prefill_attention_ws")(
            q.data_ptr(), kv.data_ptr(), sink.data_ptr(), sink.numel(), dt, B, T, H, D, S, float(softmax_scale),
            int(tile_size), None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), out.data_ptr(), st)
    _lib.check(rc, "aekv_tiled_prefill_attention")
    return out


def _tiled_checks(q, kv, sink, tile_size) -> None:
    """The reference's checks in its order, each with its message (raises on the first failure)."""
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
    # (.contiguous() as the reference wrapper, sparse_attention.py:37-39; a no-op on contiguous views)
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
