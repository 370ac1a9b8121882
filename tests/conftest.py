"""Shared test setup: import paths, the `gpu` marker, and input helpers.

CPU tests (`-m "not gpu"`) pin the oracle (oracle/) against known answers, library routines and
invariants, and check the C ABI and host-side validation without touching a GPU.  GPU tests
(`-m gpu`) compare libaetherkv on the device with the oracle on identical bytes.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "deepseek-v4-codebase_amd"
for p in (PKG_DIR, ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built libaetherkv.so")


def has_gpu() -> bool:
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def dev():
    if not has_gpu():
        pytest.skip("no HIP device")
    import aetherkv._lib as L

    if not L.available():
        pytest.fail("libaetherkv.so is not built: GPU tests must run the native library")
    return torch.device("cuda:0")


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """bf16/fp16 tensor -> uint16 numpy bit pattern (host copy)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def to_np_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().float().numpy()


def randn_outliers(shape, seed: int, dtype=torch.bfloat16, outlier_frac: float = 0.02, factor: float = 8.0,
                   device="cpu") -> torch.Tensor:
    """N(0,1) with round(frac * C) channels of the flattened trailing (H*D) axis scaled by `factor`."""
    from aetherkv.synthetic import normal_with_outliers

    return normal_with_outliers(shape, seed, dtype=dtype, outlier_frac=outlier_frac, factor=factor, device=device)
