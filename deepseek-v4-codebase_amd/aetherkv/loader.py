"""Extension loader — drop-in for aether_kernels/loader.py:24-157 on ROCm.

The reference JIT-compiles CUDA with nvcc (loader.py:106-157); here libaetherkv.so is built ahead
of time with hipcc for gfx950 (``aetherkv.build``) and loaded through ctypes.

* ``cuda_build_environment()`` returns the reference's 7 keys (tests/test_cuda_loader.py:12-22);
  on ROCm ``cuda_home`` is the ROCm root and ``nvcc`` the hipcc that builds the library.
* ``cuda_extension_unavailable_reason(require_device=False)`` is ``None`` when the library is built
  (and, with ``require_device``, a HIP device is visible).
* ``load_aether_cuda_kernels()`` returns an object exposing the four kernel functions with the
  pybind module's calling convention (bindings.cpp:124-141).
"""
from __future__ import annotations

import os
import shutil
from functools import lru_cache
from pathlib import Path
from types import SimpleNamespace
from typing import Dict, Optional

import torch

from . import _lib
from . import sparse_attention as _sa


def _rocm_home() -> Optional[str]:
    try:
        from torch.utils.cpp_extension import ROCM_HOME
    except Exception:  # pragma: no cover
        ROCM_HOME = None
    home = ROCM_HOME or os.environ.get("ROCM_PATH")
    if home is None and Path("/opt/rocm").exists():
        home = "/opt/rocm"
    return home


def cuda_build_environment() -> Dict[str, object]:
    home = _rocm_home()
    hipcc = shutil.which("hipcc") or (str(Path(home) / "bin" / "hipcc") if home and (Path(home) / "bin" / "hipcc").exists() else None)
    return {
        "torch_cuda_built": bool(torch.backends.cuda.is_built() and torch.version.hip is not None),
        "torch_cuda_available": torch.cuda.is_available(),
        "cuda_home": home,
        "nvcc": hipcc,
        "conda_target_include": None,
        "conda_target_lib": None,
        "cuda_runtime_lib": None,
    }


def cuda_extension_unavailable_reason(require_device: bool = False) -> Optional[str]:
    env = cuda_build_environment()
    if not env["torch_cuda_built"]:
        return "PyTorch was built without ROCm/HIP support."
    if require_device and not env["torch_cuda_available"]:
        return "No HIP device is available for executing the custom kernels."
    if not _lib.available():
        return f"libaetherkv.so is not built ({_lib.LIB_PATH}); run `python -m aetherkv.build`."
    return None


@lru_cache(maxsize=1)
def load_aether_cuda_kernels(verbose: bool = False, build_directory: Optional[str] = None):
    reason = cuda_extension_unavailable_reason(require_device=False)
    if reason is not None:
        raise RuntimeError(f"Aether HIP kernels are unavailable: {reason}")
    lib = _lib.lib()
    if verbose:
        print(f"[aetherkv] loaded {_lib.LIB_PATH} ({lib.aekv_version().decode()})")
    return SimpleNamespace(
        sparse_sink_attention=_sa._ext_sparse_sink_attention,
        tiled_prefill_attention=_sa._ext_tiled_prefill_attention,
        csa_indexer_topk=_sa._ext_csa_indexer_topk,
        hca_compress=_sa._ext_hca_compress,
        library_path=str(_lib.LIB_PATH),
    )
