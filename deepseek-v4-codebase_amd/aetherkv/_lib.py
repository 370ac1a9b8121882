"""ctypes binding of libaetherkv.so (the C ABI declared in include/aetherkv.h).

Torch tensors enter the ABI only as raw device pointers (``tensor.data_ptr()``), int64 sizes and
the current HIP stream handle.  A non-zero status becomes ``ValueError`` (AEKV_ERR_VALUE) or
``RuntimeError`` (everything else) carrying the library's message, matching the reference's
split between the quantiser's ``ValueError`` (turbo_quant.py:58-59, :98-99) and the extension's
``TORCH_CHECK`` ``RuntimeError`` (bindings.cpp:5-9).

There is no fallback: if the library is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libaetherkv.so"

# aekv_status
OK, ERR_VALUE, ERR_SHAPE, ERR_DTYPE, ERR_ALIGN, ERR_WORKSPACE, ERR_HIP, ERR_UNSUPPORTED = range(8)
# aekv_dtype
F32, F16, BF16, I32, I64 = range(5)
# aekv_index_mode
INDEX_MODES = {"softplus": 0, "raw": 1, "relu_w": 2}

TORCH_TO_AEKV = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.int32: I32, torch.int64: I64}

SYMBOLS = (
    "aekv_version", "aekv_last_error", "aekv_max_head_dim", "aekv_max_topk", "aekv_tq_diag", "aekv_wht",
    "aekv_tq_encode", "aekv_tq_decode", "aekv_csa_indexer_workspace_size", "aekv_csa_indexer_topk",
    "aekv_csa_indexer_topk_quant", "aekv_sparse_sink_attention", "aekv_quant_attention_workspace_size",
    "aekv_quant_sink_attention", "aekv_hca_compress", "aekv_tiled_prefill_attention", "aekv_set_generic_kernels",
    "aekv_set_flash_rows", "aekv_emit_block", "aekv_csa_prefill_indexer_topk_quant", "aekv_quant_prefill_workspace_size",
    "aekv_quant_prefill_attention", "aekv_rope_rmsnorm", "aekv_csa_indexer_topk_quant_noalloc",
    "aekv_csa_decode_workspace_size", "aekv_csa_decode_quant", "aekv_sparse_sink_attention_ws",
    "aekv_tiled_prefill_attention_ws", "aekv_sink_attention_workspace_size",
)

# size of the static device scratch behind aekv_csa_indexer_topk_quant_noalloc (AEKV_STATIC_SCRATCH_BYTES)
STATIC_SCRATCH_BYTES = 32 << 20

_lib: Optional[ctypes.CDLL] = None


class LibraryUnavailable(RuntimeError):
    pass


def available() -> bool:
    return LIB_PATH.exists()


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise LibraryUnavailable(
            f"libaetherkv.so not found at {LIB_PATH}; build it with `python -m aetherkv.build` "
            "(or __graft_entry__.build())")
    L = ctypes.CDLL(str(LIB_PATH))
    P, I64_, I32_, SZ, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t, ctypes.c_float
    sig = {
        "aekv_version": ([], ctypes.c_char_p),
        "aekv_last_error": ([], ctypes.c_char_p),
        "aekv_max_head_dim": ([], I32_),
        "aekv_max_topk": ([], I32_),
        "aekv_set_generic_kernels": ([ctypes.c_int], ctypes.c_int),
        "aekv_set_flash_rows": ([ctypes.c_int], ctypes.c_int),
        "aekv_tq_diag": ([I64_, I32_, P], ctypes.c_int),
        "aekv_wht": ([P, I32_, I64_, I32_, P, P], ctypes.c_int),
        "aekv_tq_encode": ([P, I32_, I64_, I32_, I32_, P, P, P, P], ctypes.c_int),
        "aekv_tq_decode": ([P, P, I64_, I32_, I32_, P, P, I32_, P], ctypes.c_int),
        "aekv_csa_indexer_workspace_size": ([I64_, I64_, I32_], SZ),
        "aekv_csa_indexer_topk": ([P, P, P, P, I64_, I64_, I32_, I32_, I32_, I32_, P, SZ, P, P, P], ctypes.c_int),
        "aekv_csa_indexer_topk_quant": ([P, P, P, P, P, P, I64_, I64_, I32_, I32_, I32_, I32_, I32_, P, SZ, P, P, P],
                                        ctypes.c_int),
        "aekv_sparse_sink_attention": ([P, P, P, I32_, P, I64_, I32_, I64_, I64_, I64_, I64_, I64_, I64_, F, P, P],
                                       ctypes.c_int),
        "aekv_quant_attention_workspace_size": ([I64_, I64_, I64_, I64_, I64_], SZ),
        "aekv_quant_sink_attention": ([P, P, P, P, P, P, P, I64_, I64_, I64_, I64_, I64_, I64_, I32_, F, P, SZ, P, P],
                                      ctypes.c_int),
        "aekv_hca_compress": ([P, P, I32_, I64_, I64_, I64_, P, P], ctypes.c_int),
        "aekv_emit_block": ([P, P, P, I64_, I64_, I32_, I32_, P, P, P, F, I32_, P, P, P, I64_, P, P], ctypes.c_int),
        "aekv_csa_indexer_topk_quant_noalloc": ([P, P, P, P, P, P, I64_, I64_, I32_, I32_, I32_, I32_, I32_, P, P, P],
                                                ctypes.c_int),
        "aekv_csa_decode_workspace_size": ([I64_, I64_, I32_, I64_, I64_, I64_], SZ),
        "aekv_csa_decode_quant": ([P, P, P, P, P, P, I64_, I64_, I32_, I32_, I32_, I32_, I32_, P, P, P, P, P, P, I64_,
                                   I64_, I64_, I32_, F, P, SZ, P, P, P, P], ctypes.c_int),
        "aekv_csa_prefill_indexer_topk_quant": (
            [P, P, P, P, P, P, I64_, I64_, I64_, I32_, I32_, I32_, I32_, I32_, P, SZ, P, P, P], ctypes.c_int),
        "aekv_quant_prefill_workspace_size": ([I64_, I64_, I64_, I64_, I64_], SZ),
        "aekv_rope_rmsnorm": ([P, I64_, I32_, I32_, P, I32_, P, I32_, P, F, P, P], ctypes.c_int),
        "aekv_quant_prefill_attention": (
            [P, P, P, P, P, P, P, P, P, P, I64_, I64_, I64_, I64_, I64_, I64_, I64_, I32_, F, P, SZ, P, P], ctypes.c_int),
        "aekv_tiled_prefill_attention": ([P, P, P, I64_, I32_, I64_, I64_, I64_, I64_, I64_, F, I32_, P, P],
                                         ctypes.c_int),
        "aekv_sparse_sink_attention_ws": (
            [P, P, P, I32_, P, I64_, I32_, I64_, I64_, I64_, I64_, I64_, I64_, F, P, SZ, P, P], ctypes.c_int),
        "aekv_tiled_prefill_attention_ws": (
            [P, P, P, I64_, I32_, I64_, I64_, I64_, I64_, I64_, F, I32_, P, SZ, P, P], ctypes.c_int),
        "aekv_sink_attention_workspace_size": ([I32_, I64_, I64_, I64_, I64_, I64_, I64_], SZ),
    }
    for name, (argtypes, restype) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = argtypes
        fn.restype = restype
    _lib = L
    return _lib


_hot: dict = {}


def hot(name: str):
    """The entry point `name` for calls made once per token: the CPython fast-call function of
    aetherkv._fastcall when that module is built (same arguments as plain ints / floats / None),
    else the ctypes function.  The library is loaded through ctypes first, so both use one copy."""
    fn = _hot.get(name)
    if fn is None:
        L = lib()
        try:
            from . import _fastcall  # noqa: WPS433 (built next to libaetherkv.so)

            fn = getattr(_fastcall, name)
        except (ImportError, AttributeError):
            fn = getattr(L, name)
        _hot[name] = fn
    return fn


def check(rc: int, what: str) -> None:
    if rc == OK:
        return
    msg = lib().aekv_last_error().decode("utf-8", "replace") or f"{what} failed with status {rc}"
    if rc == ERR_VALUE:
        raise ValueError(msg)
    raise RuntimeError(msg)


def ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def raw_stream(device: torch.device) -> int:
    """The current HIP stream of `device` as an integer handle (no Stream object is built)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


class _Nothing:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NOTHING = _Nothing()


def on_device(device: torch.device):
    """Context making `device` current: nothing to do when it already is (the common case)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _NOTHING
    return torch.cuda.device(device)


# Split workspaces of the drop-in attention calls, one per (device, stream): calls on one stream run
# in order, so each reuses the previous call's buffer.  Not grown while a graph is being captured
# (the buffer would come from the graph's private pool): such calls get a buffer of their own.
_ws_cache: dict = {}


def workspace(nbytes: int, device: torch.device, stream: int) -> Optional[torch.Tensor]:
    if nbytes <= 0:
        return None
    key = (device.index, stream)
    buf = _ws_cache.get(key)
    if buf is not None and buf.numel() >= nbytes:
        return buf
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    buf = torch.empty(max(nbytes, 2 * buf.numel() if buf is not None else 0), dtype=torch.uint8, device=device)
    _ws_cache[key] = buf
    return buf


def require_device(name: str, *tensors: Optional[torch.Tensor]) -> None:
    """The product path runs on HIP devices only; CPU tensors are rejected loudly."""
    for t in tensors:
        if t is not None and not t.is_cuda:  # (is_cuda: no device object built per tensor)
            raise RuntimeError(f"{name} must be a HIP device tensor (got {t.device}); aetherkv has no CPU path")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return TORCH_TO_AEKV[t.dtype]
    except KeyError as exc:
        raise RuntimeError(f"unsupported dtype {t.dtype}") from exc


def aligned(t: torch.Tensor, nbytes: int) -> torch.Tensor:
    """Contiguous tensor whose data pointer is a multiple of `nbytes` (copies only when needed)."""
    t = t.contiguous()
    if t.numel() and t.data_ptr() % nbytes:
        t = t.clone()
    return t
