"""aekv_csa_indexer_topk_quant_noalloc: the indexer with its scratch in a static device array.

Called through the C ABI with raw pointers, it must return exactly what the workspace entry point
aekv_csa_indexer_topk_quant returns on the same inputs (same kernels, bit for bit), on two calls in
a row, the second smaller than the first (the array keeps the first call's contents).  A launch
whose workspace exceeds the array is refused before any device work.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

import aetherkv._lib as L
from aetherkv import PolarQuant
from aetherkv.synthetic import normal, normal_with_outliers


def _call_both(dev, B, S, IH, IC, bits, k, seed, valid=None, mode=0):
    pq = PolarQuant(bits)
    codes, scale = pq.encode(normal_with_outliers((B, S, IC), seed, device=dev, trailing_dims=1))
    q = normal((B, IH, IC), seed + 1, dtype=torch.float32).to(dev)
    w = normal((B, IH), seed + 2, dtype=torch.float32).to(dev)
    diag = pq._diag(IC, dev)
    v = None if valid is None else torch.tensor(valid, dtype=torch.int32, device=dev)
    lib = L.lib()
    st = L.stream_of(q)
    ws = torch.empty(lib.aekv_csa_indexer_workspace_size(B, S, k), dtype=torch.uint8, device=dev)
    idx_ws = torch.full((B, k), -7, dtype=torch.int64, device=dev)
    sc_ws = torch.full((B, k), -7.0, dtype=torch.float32, device=dev)
    rc = lib.aekv_csa_indexer_topk_quant(L.ptr(q), L.ptr(w), L.ptr(codes), L.ptr(scale), L.ptr(diag), L.ptr(v), B, S,
                                         IH, IC, bits, k, mode, L.ptr(ws), ws.numel(), L.ptr(idx_ws), L.ptr(sc_ws), st)
    assert rc == L.OK, lib.aekv_last_error()
    idx_na = torch.full((B, k), -9, dtype=torch.int64, device=dev)
    sc_na = torch.full((B, k), -9.0, dtype=torch.float32, device=dev)
    rc = lib.aekv_csa_indexer_topk_quant_noalloc(L.ptr(q), L.ptr(w), L.ptr(codes), L.ptr(scale), L.ptr(diag),
                                                 L.ptr(v), B, S, IH, IC, bits, k, mode, L.ptr(idx_na), L.ptr(sc_na),
                                                 st)
    assert rc == L.OK, lib.aekv_last_error()
    torch.cuda.synchronize()
    return idx_ws, sc_ws, idx_na, sc_na


@pytest.mark.gpu
def test_noalloc_indexer_equals_workspace_entry_point_twice(dev):
    # first call: cfg5's launch (64 rows x 65536 4-bit keys, 17.8 MB of scratch); second: smaller and
    # ragged, so stale order keys and slot maxima of the first call sit in the array
    print("noalloc indexer: cfg5 launch", flush=True)
    a = _call_both(dev, 64, 65536, 4, 64, 4, 256, 4)
    assert torch.equal(a[0], a[2]) and torch.equal(a[1], a[3])
    assert bool((a[2] >= 0).all())
    print("noalloc indexer: smaller ragged launch", flush=True)
    b = _call_both(dev, 5, 3001, 4, 64, 8, 64, 9, valid=[3001, 0, 17, 1500, 64], mode=1)
    assert torch.equal(b[0], b[2]) and torch.equal(b[1], b[3])
    assert bool((b[2][1] == -1).all()) and int((b[2][2] >= 0).sum()) == 17


def test_noalloc_indexer_rejects_launches_beyond_the_static_scratch():
    # host-side: refused with a clear message before any HIP call (runs without a GPU)
    lib = L.lib()
    B, S, k = 64, 131072, 256
    assert lib.aekv_csa_indexer_workspace_size(B, S, k) > L.STATIC_SCRATCH_BYTES
    fake = ctypes.c_void_p(256)
    rc = lib.aekv_csa_indexer_topk_quant_noalloc(fake, fake, fake, fake, fake, None, B, S, 4, 64, 4, k, 0, fake, None,
                                                 None)
    assert rc == L.ERR_UNSUPPORTED
    assert b"static" in lib.aekv_last_error()
    # argument errors come first, as in the workspace entry point
    rc = lib.aekv_csa_indexer_topk_quant_noalloc(fake, fake, fake, fake, fake, None, B, S, 4, 64, 5, k, 0, fake, None,
                                                 None)
    assert rc == L.ERR_VALUE
    # an empty launch does nothing
    assert lib.aekv_csa_indexer_topk_quant_noalloc(None, None, None, None, None, None, 0, S, 4, 64, 4, k, 0, None, None,
                                                   None) == L.OK
