"""GPU parity of the drop-in attention entry points on their matrix-core path (head_dim 128,
bf16/fp16) against the oracle.

sparse_sink_attention and tiled_prefill_attention at head_dim 128 in bf16/fp16 run on the matrix
cores; the tolerance is the reference's own for its CUDA kernel against the torch backend,
atol = rtol = 5e-3 for fp16/bf16 (tests/test_cuda_runtime.py:33-35 in the reference).  The oracle is
aether_pipeline/serving.py:99-130 in fp32 with the CUDA kernel's skip of out-of-range indices.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import aetherkv._lib as L
import oracle as O
from aetherkv import sparse_sink_attention, tiled_prefill_attention
from conftest import to_np_f32

pytestmark = pytest.mark.gpu

TOL = 5e-3


def _close(got: torch.Tensor, want: np.ndarray):
    np.testing.assert_allclose(to_np_f32(got), want, rtol=TOL, atol=TOL)


def _inputs(seed, B, T, H, S, K, dtype, idx_dtype=torch.int64, lo=0, hi=None, qscale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, T, H, 128, generator=g) * qscale).to(dtype)
    kv = torch.randn(B, S, 2, 128, generator=g).to(dtype)
    topk = torch.randint(lo, S if hi is None else hi, (B, T, K), generator=g, dtype=idx_dtype)
    sink = torch.randn(H, generator=g).to(dtype)
    return q, kv, topk, sink


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("H,K", [(16, 64), (16, 1), (8, 31), (16, 100), (20, 257), (3, 520)])
def test_sparse_matrix_core_shapes(dev, dtype, idx_dtype, H, K):
    # K covers one partial group, 2 / 4 / 8 waves per workgroup and several groups per wave; H = 20
    # takes two head groups (the second partial), H = 3 and 8 partial columns
    q, kv, topk, sink = _inputs(11 + H + K, 3, 5, H, 700, K, dtype, idx_dtype)
    got = sparse_sink_attention(q.to(dev), kv.to(dev), topk.to(dev), sink.to(dev), 128 ** -0.5)
    assert got.dtype == dtype and got.shape == q.shape
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), topk.numpy(), to_np_f32(sink), 128 ** -0.5)
    _close(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sparse_matrix_core_invalid_duplicate_and_empty(dev, dtype):
    q, kv, topk, sink = _inputs(21, 2, 4, 16, 90, 150, dtype, lo=-20, hi=110)  # ~30% skipped
    topk[0, 1] = -1                                                          # no valid source
    topk[1, 2] = 7                                                           # one source, 150 times
    sink_s = sink[:1].clone()                                                # scalar sink
    got = sparse_sink_attention(q.to(dev), kv.to(dev), topk.to(dev), sink_s.to(dev), 0.09)
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), topk.numpy(), to_np_f32(sink_s), 0.09)
    _close(got, want)
    assert not bool(got[0, 1].float().abs().sum())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sparse_matrix_core_peaked_logits_and_sink(dev, dtype):
    # large logits (a few keys dominate: the running maximum moves between groups) and sinks that
    # dominate some heads
    q, kv, topk, sink = _inputs(23, 2, 3, 16, 500, 384, dtype, qscale=4.0)
    sink = (torch.arange(16) - 8.0).to(dtype) * 3.0
    got = sparse_sink_attention(q.to(dev), kv.to(dev), topk.to(dev), sink.to(dev), 128 ** -0.5)
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), topk.numpy(), to_np_f32(sink), 128 ** -0.5)
    _close(got, want)


def test_sparse_matrix_core_no_sources(dev):
    # K = 0: every output is zero (the sink alone)
    q, kv, _, sink = _inputs(25, 2, 3, 16, 40, 1, torch.bfloat16)
    topk = torch.empty(2, 3, 0, dtype=torch.int64)
    got = sparse_sink_attention(q.to(dev), kv.to(dev), topk.to(dev), sink.to(dev), 0.1)
    assert not bool(got.float().abs().sum())


def test_sparse_matrix_core_matches_fp32_path(dev):
    # the same inputs through the fp32 VALU kernel (inputs widened exactly): the two paths agree to
    # the bf16 output rounding plus the weights' rounding
    q, kv, topk, sink = _inputs(27, 2, 8, 16, 1000, 200, torch.bfloat16)
    got = sparse_sink_attention(q.to(dev), kv.to(dev), topk.to(dev), sink.to(dev), 128 ** -0.5)
    ref = sparse_sink_attention(q.float().to(dev), kv.float().to(dev), topk.to(dev), sink.float().to(dev), 128 ** -0.5)
    np.testing.assert_allclose(to_np_f32(got), to_np_f32(ref), rtol=TOL, atol=TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,S", [(1, 1, 640), (4, 1, 200), (2, 3, 33)])
def test_tiled_prefill_matrix_core_model_calls(dev, dtype, B, T, S):
    # modeling.py:322,534 calls tiled_prefill_attention per target: q [B, 1, H, D] over the
    # target's [blocks; window] sources stacked as K = V
    g = torch.Generator().manual_seed(31 + S)
    q = torch.randn(B, T, 16, 128, generator=g).to(dtype)
    src = torch.randn(B, S, 128, generator=g).to(dtype)
    kv = torch.stack([src, src], dim=2)
    sink = torch.randn(16, generator=g).to(dtype)
    got = tiled_prefill_attention(q.to(dev), kv.to(dev), sink.to(dev), 128 ** -0.5, tile_size=256)
    idx = np.broadcast_to(np.arange(S), (B, T, S))
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), idx, to_np_f32(sink), 128 ** -0.5)
    _close(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_tiled_prefill_matrix_core_prefill_shape(dev, dtype):
    # T = 256 targets over S = 8192 sources, 16 heads, separate K and V
    g = torch.Generator().manual_seed(37)
    B, T, H, S = 1, 256, 16, 8192
    q = torch.randn(B, T, H, 128, generator=g).to(dtype)
    kv = torch.randn(B, S, 2, 128, generator=g).to(dtype)
    sink = torch.randn(H, generator=g).to(dtype)
    got = tiled_prefill_attention(q.to(dev), kv.to(dev), sink.to(dev), 128 ** -0.5, tile_size=256)
    idx = np.broadcast_to(np.arange(S), (B, T, S))
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), idx, to_np_f32(sink), 128 ** -0.5, threads=16)
    _close(got, want)


@pytest.mark.parametrize("B,T,S", [(1, 1, 640), (1, 256, 4096)])
def test_unsplit_entry_points(dev, B, T, S):
    # the reference-signature C entry points (no workspace: one workgroup per target, or per row
    # block, over all its sources) against the oracle, at shapes the wrappers split
    assert L.lib().aekv_sink_attention_workspace_size(L.BF16, B, T, 16, 128, S, -1) > 0
    g = torch.Generator().manual_seed(41 + T)
    q = torch.randn(B, T, 16, 128, generator=g).to(torch.bfloat16)
    kv = torch.randn(B, S, 2, 128, generator=g).to(torch.bfloat16)
    sink = torch.randn(16, generator=g).to(torch.bfloat16)
    topk = torch.randint(0, S, (B, T, S), generator=g, dtype=torch.int32)
    qd, kvd, sd, td = q.to(dev), kv.to(dev), sink.to(dev), topk.to(dev)
    out_d = torch.empty_like(qd)
    out_s = torch.empty_like(qd)
    with torch.cuda.device(dev):
        L.check(L.lib().aekv_tiled_prefill_attention(L.ptr(qd), L.ptr(kvd), L.ptr(sd), 16, L.BF16, B, T, 16, 128, S,
                                                     128 ** -0.5, 256, L.ptr(out_d), L.stream_of(qd)), "tiled")
        L.check(L.lib().aekv_sparse_sink_attention(L.ptr(qd), L.ptr(kvd), L.ptr(td), L.I32, L.ptr(sd), 16, L.BF16, B,
                                                   T, 16, 128, S, S, 128 ** -0.5, L.ptr(out_s), L.stream_of(qd)),
                "sparse")
    torch.cuda.synchronize()
    want_d = O.sink_attention(to_np_f32(q), to_np_f32(kv), np.broadcast_to(np.arange(S), (B, T, S)),
                              to_np_f32(sink), 128 ** -0.5, threads=16)
    _close(out_d, want_d)
    if T == 1:
        want_s = O.sink_attention(to_np_f32(q), to_np_f32(kv), topk.numpy(), to_np_f32(sink), 128 ** -0.5)
        _close(out_s, want_s)
        # and the wrapper (split into pieces) on the same call
        _close(sparse_sink_attention(qd, kvd, td, sd, 128 ** -0.5), want_s)


def test_misaligned_views_take_the_valu_kernel(dev):
    # q and kv views one element into their storage are not 16-byte aligned: the call falls back
    # to the VALU kernel (the wrapper keeps contiguous views as they are), same results
    g = torch.Generator().manual_seed(43)
    q0 = torch.randn(2 * 3 * 16 * 128 + 1, generator=g).to(torch.bfloat16)
    kv0 = torch.randn(2 * 90 * 2 * 128 + 1, generator=g).to(torch.bfloat16)
    q = q0[1:].view(2, 3, 16, 128)
    kv = kv0[1:].view(2, 90, 2, 128)
    topk = torch.randint(0, 90, (2, 3, 70), generator=g)
    sink = torch.randn(16, generator=g).to(torch.bfloat16)
    qd, kvd = q0.to(dev)[1:].view(2, 3, 16, 128), kv0.to(dev)[1:].view(2, 90, 2, 128)
    assert qd.data_ptr() % 16 != 0
    got = sparse_sink_attention(qd, kvd, topk.to(dev), sink.to(dev), 128 ** -0.5)
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), topk.numpy(), to_np_f32(sink), 128 ** -0.5)
    _close(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_tiled_prefill_flash_many_heads_scalar_sink(dev, dtype):
    # 20 heads (row blocks of 64 cross target boundaries), scalar sink, S not a multiple of the tile
    g = torch.Generator().manual_seed(47)
    B, T, H, S = 2, 7, 20, 1000
    q = torch.randn(B, T, H, 128, generator=g).to(dtype)
    kv = torch.randn(B, S, 2, 128, generator=g).to(dtype)
    sink = torch.randn(1, generator=g).to(dtype)
    got = tiled_prefill_attention(q.to(dev), kv.to(dev), sink.to(dev), 0.1)
    idx = np.broadcast_to(np.arange(S), (B, T, S))
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), idx, to_np_f32(sink), 0.1)
    _close(got, want)


def test_split_calls_in_a_graph(dev):
    # the split workspace (taken from torch's allocator inside the capture) and the combine kernel
    # replayed from a HIP graph, eager work between replays, every replay against the eager result
    g = torch.Generator().manual_seed(53)
    q = torch.randn(1, 1, 16, 128, generator=g).to(torch.bfloat16).to(dev)
    src = torch.randn(1, 640, 128, generator=g).to(torch.bfloat16)
    kv = torch.stack([src, src], dim=2).to(dev)
    sink = torch.randn(16, generator=g).to(torch.bfloat16).to(dev)
    qs = torch.randn(1, 4, 16, 128, generator=g).to(torch.bfloat16).to(dev)
    kvs = torch.randn(1, 3000, 2, 128, generator=g).to(torch.bfloat16).to(dev)
    topk = torch.randint(0, 3000, (1, 4, 600), generator=g, dtype=torch.int32).to(dev)
    want_d = tiled_prefill_attention(q, kv, sink, 128 ** -0.5)
    want_s = sparse_sink_attention(qs, kvs, topk, sink, 128 ** -0.5)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        tiled_prefill_attention(q, kv, sink, 128 ** -0.5)
        sparse_sink_attention(qs, kvs, topk, sink, 128 ** -0.5)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_d = tiled_prefill_attention(q, kv, sink, 128 ** -0.5)
        out_s = sparse_sink_attention(qs, kvs, topk, sink, 128 ** -0.5)
    for _ in range(3):
        out_d.zero_()
        out_s.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_d, want_d) and torch.equal(out_s, want_s)
        tiled_prefill_attention(qs, kvs, sink, 0.2)  # eager work between replays


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_no_valid_source_with_sink_minus_inf_is_zero_split_or_not(dev, dtype):
    # A target whose indices are all out of range, with the sink at -inf: the reference kernel's
    # weighted sum skips every index and writes 0 (sparse_sink_attention_cuda.cu:102-114), so every
    # route gives 0 — the split launch (the wrapper's workspace) and the unsplit C entry point —
    # while the other targets match the oracle.
    B, T, H, S, K = 1, 2, 16, 640, 640
    g = torch.Generator().manual_seed(47)
    q = torch.randn(B, T, H, 128, generator=g).to(dtype)
    kv = torch.randn(B, S, 2, 128, generator=g).to(dtype)
    topk = torch.randint(0, S, (B, T, K), generator=g, dtype=torch.int32)
    topk[0, 1] = -1                                  # target 1: no valid source
    sink = torch.full((H,), float("-inf")).to(dtype)
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), topk.numpy(), to_np_f32(sink), 128 ** -0.5)
    assert not np.abs(want[0, 1]).sum() and np.isfinite(want).all()
    qd, kvd, td, sd = q.to(dev), kv.to(dev), topk.to(dev), sink.to(dev)
    split = sparse_sink_attention(qd, kvd, td, sd, 128 ** -0.5)
    unsplit = torch.empty_like(qd)
    with torch.cuda.device(dev):
        L.check(L.lib().aekv_sparse_sink_attention(L.ptr(qd), L.ptr(kvd), L.ptr(td), L.I32, L.ptr(sd), H,
                                                   L.dtype_code(qd), B, T, H, 128, S, K, 128 ** -0.5, L.ptr(unsplit),
                                                   L.stream_of(qd)), "sparse")
    torch.cuda.synchronize()
    tol = 1e-4 if dtype == torch.float32 else TOL
    for got in (split, unsplit):
        assert torch.isfinite(got.float()).all()
        np.testing.assert_allclose(to_np_f32(got), want, rtol=tol, atol=tol)
        assert not bool(got[0, 1].float().abs().sum())


def test_quant_attention_without_sources_and_sink_minus_inf_is_zero(dev):
    # the quantised decode attention (the engine returns zeros when a step has no source,
    # aether_2b/serving.py:451-452): every selected index skipped, no window, sink -inf -> 0, in
    # one piece and split over pieces (a row of 3000 selected blocks)
    from aetherkv import PolarQuant
    from aetherkv.decode import quant_sink_attention

    pq = PolarQuant(4)
    B, H, S = 2, 12, 4000
    g = torch.Generator().manual_seed(49)
    codes, scale = pq.encode(torch.randn(B, S, 128, generator=g).to(torch.bfloat16).to(dev))
    q = torch.randn(B, 1, H, 128, generator=g).to(torch.bfloat16).to(dev)
    sink = torch.full((H,), float("-inf"), device=dev)
    for K in (100, 3000):
        sel = torch.full((B, K), -1, dtype=torch.int64, device=dev)
        sel[0] = torch.randint(0, S, (K,), generator=g).to(dev)     # row 0 has sources, row 1 none
        out = quant_sink_attention(q, codes, scale, sel, None, sink, 128 ** -0.5, quant=pq)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all(), K
        assert not bool(out[1].float().abs().sum()), K
        want = O.quant_attention(to_np_f32(q).reshape(B, H, 128), codes.cpu().numpy(), scale.cpu().numpy(),
                                 sel.cpu().numpy(), np.zeros((B, 0, 128), np.float32), to_np_f32(sink),
                                 O.diag(42, 128), 4, 128 ** -0.5)
        np.testing.assert_allclose(to_np_f32(out).reshape(B, H, 128), want, rtol=1e-2, atol=2e-3)
