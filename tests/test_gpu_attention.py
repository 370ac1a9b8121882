"""GPU parity of the attention kernels against the oracle.

Tolerances: the reference's own CUDA-vs-torch test uses atol = rtol = 5e-3 for fp16/bf16 and 1e-4
for fp32 (tests/test_cuda_runtime.py:33-35 in the reference); the quantised decode path is held to
the path's stated 1e-2 relative / 2e-3 absolute in bf16.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from aetherkv import PolarQuant, hca_compress, sparse_sink_attention, tiled_prefill_attention
from aetherkv.decode import csa_decode, hca_decode, quant_sink_attention
from aetherkv.synthetic import normal, normal_with_outliers, rope_interleaved
from conftest import to_np_f32

pytestmark = pytest.mark.gpu

QUANT_RTOL, QUANT_ATOL = 1e-2, 2e-3


def _close(got: torch.Tensor, want: np.ndarray, rtol: float, atol: float):
    np.testing.assert_allclose(to_np_f32(got), want, rtol=rtol, atol=atol)


@pytest.mark.parametrize("dtype,idx_dtype,tol", [(torch.float32, torch.int64, 1e-4), (torch.float16, torch.int32, 5e-3),
                                                 (torch.bfloat16, torch.int64, 5e-3)])
def test_sparse_sink_attention_reference_case(dev, dtype, idx_dtype, tol):
    # tests/test_cuda_runtime.py:19-35 of the reference, same shapes and seed
    torch.manual_seed(0)
    q = torch.randn(2, 5, 4, 16, dtype=dtype)
    kv = torch.randn(2, 23, 2, 16, dtype=dtype)
    topk = torch.randint(0, 23, (2, 5, 7), dtype=idx_dtype)
    sink = torch.randn(4, dtype=dtype)
    got = sparse_sink_attention(q.to(dev), kv.to(dev), topk.to(dev), sink.to(dev), 0.125)
    assert got.dtype == dtype and got.shape == q.shape
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), topk.numpy(), to_np_f32(sink), 0.125)
    _close(got, want, tol, tol)


def test_sparse_sink_attention_invalid_and_duplicate_indices(dev):
    g = torch.Generator().manual_seed(5)
    q = torch.randn(3, 2, 4, 64, generator=g).to(torch.bfloat16)
    kv = torch.randn(3, 40, 2, 64, generator=g).to(torch.bfloat16)
    topk = torch.randint(-5, 45, (3, 2, 90), generator=g)  # out-of-range entries are skipped
    topk[0, 0] = -1                                          # a row with no valid source -> zeros
    sink = torch.tensor(0.3).to(torch.bfloat16)               # scalar sink
    got = sparse_sink_attention(q.to(dev), kv.to(dev), topk.to(dev), sink.reshape(1).to(dev), 0.2)
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), topk.numpy(), to_np_f32(sink.reshape(1)), 0.2)
    _close(got, want, 5e-3, 5e-3)
    assert not bool(got[0, 0].float().abs().sum())


def test_sparse_sink_attention_report_shape(dev):
    # TECHNICAL_REPORT.md:228-235 microbenchmark shape: fp16, B=1, T=128, H=16, D=128, S=8192, top_k=64
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 128, 16, 128, generator=g).half()
    kv = torch.randn(1, 8192, 2, 128, generator=g).half()
    topk = torch.randint(0, 8192, (1, 128, 64), generator=g, dtype=torch.int32)
    sink = torch.zeros(16).half()
    got = sparse_sink_attention(q.to(dev), kv.to(dev), topk.to(dev), sink.to(dev), 128 ** -0.5)
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), topk.numpy(), to_np_f32(sink), 128 ** -0.5)
    _close(got, want, 5e-3, 5e-3)


def test_tiled_prefill_counts_sink_once(dev):
    g = torch.Generator().manual_seed(9)
    q = torch.randn(2, 5, 3, 32, generator=g).to(torch.bfloat16)
    kv = torch.randn(2, 600, 2, 32, generator=g).to(torch.bfloat16)
    sink = torch.randn(3, generator=g).to(torch.bfloat16)
    got = tiled_prefill_attention(q.to(dev), kv.to(dev), sink.to(dev), 32 ** -0.5, tile_size=256)
    idx = np.broadcast_to(np.arange(600), (2, 5, 600))
    want = O.sink_attention(to_np_f32(q), to_np_f32(kv), idx, to_np_f32(sink), 32 ** -0.5)
    _close(got, want, 5e-3, 5e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hca_compress(dev, dtype):
    g = torch.Generator().manual_seed(11)
    c = torch.randn(4, 128, 128, generator=g).to(dtype)
    z = (torch.randn(4, 128, 128, generator=g) * 2).to(dtype)
    got = hca_compress(c.to(dev), z.to(dev))
    assert got.shape == (4, 128) and got.dtype == dtype
    tol = 1e-5 if dtype == torch.float32 else 5e-3
    _close(got, O.hca_compress(to_np_f32(c), to_np_f32(z)), tol, tol)


def _quant_inputs(dev, B, H, D, S, W, bits, seed, outliers=False):
    pq = PolarQuant(bits)
    blocks = (normal_with_outliers((B, S, D), seed, trailing_dims=1) if outliers else normal((B, S, D), seed)).to(dev)
    codes, scale = pq.encode(blocks)
    q = normal((B, 1, H, D), seed + 1).to(dev)
    win = normal((B, W, D), seed + 2).to(dev)
    sink = normal((H,), seed + 3, dtype=torch.float32).to(dev)
    return pq, codes, scale, q, win, sink


def _oracle_quant(pq, codes, scale, sel, q, win, sink, sm):
    B, _, H, D = q.shape
    return O.quant_attention(to_np_f32(q).reshape(B, H, D), codes.cpu().numpy(), scale.cpu().numpy(),
                             None if sel is None else sel.cpu().numpy(), to_np_f32(win), to_np_f32(sink),
                             O.diag(42, D), pq.bits, sm)


@pytest.mark.parametrize("bits", [8, 4])
def test_quant_attention_selected_blocks(dev, bits):
    B, H, D, S, K, W = 4, 12, 128, 3000, 256, 128
    pq, codes, scale, q, win, sink = _quant_inputs(dev, B, H, D, S, W, bits, 40 + bits)
    g = torch.Generator().manual_seed(3)
    sel = torch.randint(0, S, (B, K), generator=g)
    sel[1, :10] = -1                       # skipped entries (padding)
    sel = sel.to(dev)
    sm = D ** -0.5
    got = quant_sink_attention(q, codes, scale, sel, win, sink, sm, quant=pq)
    assert got.shape == q.shape and got.dtype == torch.bfloat16
    _close(got.view(B, H, D), _oracle_quant(pq, codes, scale, sel, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)


def test_quant_attention_partial_window_and_empty(dev):
    B, H, D, S = 2, 4, 64, 50
    pq, codes, scale, q, win, sink = _quant_inputs(dev, B, H, D, S, 5, 8, 77)
    sm = 0.3
    sel = torch.randint(0, S, (B, 7)).to(dev)
    got = quant_sink_attention(q, codes, scale, sel, win, sink, sm, quant=pq)
    _close(got.view(B, H, D), _oracle_quant(pq, codes, scale, sel, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)
    # window only (no compressed block visible yet)
    got = quant_sink_attention(q, codes, scale, sel[:, :0], win, sink, sm, quant=pq)
    _close(got.view(B, H, D), _oracle_quant(pq, codes, scale, sel[:, :0], q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)
    # no sources at all -> zeros (serving.py:451-452)
    got = quant_sink_attention(q, codes, scale, sel[:, :0], None, sink, sm, quant=pq)
    assert not bool(got.float().abs().sum())


def test_config4_hca_decode_4bit(dev):
    # benchmark configuration cfg4: B=32, 2048 blocks (compression 128, RoPE at block end, theta 1e4), 4-bit, window 128
    B, H, D, S, W = 32, 12, 128, 2048, 128
    pq = PolarQuant(4)
    raw = normal((B, S, D), 3).to(dev)
    pos = torch.arange(S, device=dev) * 128 + 127
    blocks = rope_interleaved(raw, pos, 64, 10000.0)
    codes, scale = pq.encode(blocks)
    q = normal((B, 1, H, D), 4).to(dev)
    win = normal((B, W, D), 5).to(dev)
    sink = normal((H,), 6, dtype=torch.float32).to(dev)
    sm = D ** -0.5
    got = hca_decode(q, codes, scale, win, sink, sm, kv_quant=pq)
    _close(got.view(B, H, D), _oracle_quant(pq, codes, scale, None, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)


@pytest.mark.parametrize("bits", [4, 8])
def test_quant_attention_more_splits_than_a_combine_chunk(dev, bits):
    # 2 rows of 5000 blocks + 128 window rows: 11 pieces of 512 sources per row, so the split
    # combine merges two chunks (8 + 3); in row 1 every selected entry past the first 600 is
    # skipped, so most of its pieces hold no source (max -inf, sum 0)
    B, H, D, S, W = 2, 12, 128, 5000, 128
    pq, codes, scale, q, win, sink = _quant_inputs(dev, B, H, D, S, W, bits, 60 + bits)
    sm = D ** -0.5
    got = hca_decode(q, codes, scale, win, sink, sm, kv_quant=pq)
    _close(got.view(B, H, D), _oracle_quant(pq, codes, scale, None, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)
    g = torch.Generator().manual_seed(61)
    sel = torch.randint(0, S, (B, S), generator=g)
    sel[1, 600:] = -1
    sel = sel.to(dev)
    got = quant_sink_attention(q, codes, scale, sel, win, sink, sm, quant=pq)
    _close(got.view(B, H, D), _oracle_quant(pq, codes, scale, sel, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)


def test_split_rows_whatever_the_workspace_holds(dev):
    # 1516 sources per row: two pieces and the combine.  The workspace's prior contents must not
    # matter: zeros, all ones and random bytes give bit-identical results, equal to the oracle.
    from aetherkv.decode import attention_workspace
    B, H, D, S, W, bits = 3, 12, 128, 1500, 16, 4
    pq, codes, scale, q, win, sink = _quant_inputs(dev, B, H, D, S, W, bits, 77)
    sm = D ** -0.5
    ws = attention_workspace(B, H, D, S, W, dev)
    outs = []
    for fill in ("zeros", "ones", "random", "random"):
        if fill == "zeros":
            ws.zero_()
        elif fill == "ones":
            ws.fill_(255)
        else:
            ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, device=dev))
        print(f"split merge, workspace {fill}", flush=True)
        outs.append(quant_sink_attention(q, codes, scale, None, win, sink, sm, quant=pq, workspace=ws))
        torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    _close(outs[0].view(B, H, D), _oracle_quant(pq, codes, scale, None, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)


@pytest.mark.parametrize("B,H", [(3, 5), (1, 1)])
def test_split_rows_odd_row_head_count(dev, B, H):
    # 1516 sources per row: three pieces of 512 and the combine, whose workgroups hold two
    # (row, head) pairs; an odd rows x heads leaves the last workgroup's second pair empty
    D, S, W, bits = 128, 1500, 16, 4
    pq, codes, scale, q, win, sink = _quant_inputs(dev, B, H, D, S, W, bits, 91 + H)
    sm = D ** -0.5
    print(f"split rows B={B} H={H}", flush=True)
    got = hca_decode(q, codes, scale, win, sink, sm, kv_quant=pq)
    _close(got.view(B, H, D), _oracle_quant(pq, codes, scale, None, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)


@pytest.mark.parametrize("S,W,bits", [
    (0, 5, 4),      # window only
    (37, 0, 8),     # blocks only, one partial group
    (70, 3, 8),     # one piece holding blocks, then window rows, in one group
    (1000, 40, 4),  # two pieces, the second holding the last blocks and the window
    (1023, 1, 4),   # the one window row alone in the second piece's last group
    (600, 200, 8),  # window rows spread over several groups and waves
])
def test_every_block_decode_rows_edges(dev, S, W, bits):
    # decode rows over every block with no per-row counts take the dense kernel: every lane issues
    # its loads whatever its source, reading past the buffer ranges (zeros) where it has none
    B, H, D = 3, 12, 128
    pq, codes, scale, q, win, sink = _quant_inputs(dev, B, H, D, max(S, 1), max(W, 1), bits, 300 + S + W)
    codes, scale = codes[:, :S].contiguous(), scale[:, :S].contiguous()
    win = win[:, :W].contiguous() if W else None
    sm = D ** -0.5
    print(f"every-block decode S={S} W={W} bits={bits}", flush=True)
    got = quant_sink_attention(q, codes, scale, None, win, sink, sm, quant=pq)
    want = O.quant_attention(to_np_f32(q).reshape(B, H, D), codes.cpu().numpy(), scale.cpu().numpy(), None,
                             np.zeros((B, 0, D), np.float32) if win is None else to_np_f32(win), to_np_f32(sink),
                             O.diag(42, D), bits, sm)
    _close(got.view(B, H, D), want, QUANT_RTOL, QUANT_ATOL)


@pytest.mark.parametrize("S", [130400, 130900])
def test_quant_attention_most_pieces(dev, S):
    # one row, S blocks + 128 window rows in pieces of 512: 255 pieces, and 256 (the launch limit);
    # the combine merges 32 chunks of 8 pieces
    B, H, D, W, bits = 1, 12, 128, 128, 4
    pq, codes, scale, q, win, sink = _quant_inputs(dev, B, H, D, S, W, bits, 88)
    sm = D ** -0.5
    print(f"quant attention {S + W} sources", flush=True)
    got = hca_decode(q, codes, scale, win, sink, sm, kv_quant=pq)
    _close(got.view(B, H, D), _oracle_quant(pq, codes, scale, None, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)


def test_config3_csa_decode_end_to_end(dev):
    # benchmark configuration cfg3: B=8, 16384 blocks, 8-bit codes, indexer 4x64 softplus, top-256 + window 128 + sink
    B, H, D, S, W, IH, IC = 8, 12, 128, 16384, 128, 4, 64
    pq = PolarQuant(8)
    pq_idx = PolarQuant(8)
    kv_codes, kv_scale = pq.encode(normal((B, S, D), 2).to(dev))
    ix_codes, ix_scale = pq_idx.encode(normal((B, S, IC), 12).to(dev))
    q = normal((B, 1, H, D), 22).to(dev)
    index_q = normal((B, IH, IC), 32, dtype=torch.float32).to(dev)
    index_w = normal((B, IH), 42, dtype=torch.float32).to(dev)
    win = normal((B, W, D), 52).to(dev)
    sink = normal((H,), 62, dtype=torch.float32).to(dev)
    sm = D ** -0.5
    out, idx = csa_decode(q, index_q, index_w, ix_codes, ix_scale, kv_codes, kv_scale, win, sink, sm, kv_quant=pq,
                          index_quant=pq_idx, top_k=256)
    assert idx.shape == (B, 256) and out.shape == q.shape
    # selection vs the oracle (set equality up to fp32 near-ties) ...
    from test_gpu_indexer import w_act
    from topk_check import assert_topk_matches, score_error_bound

    keys = O.decode(ix_codes.cpu().numpy(), ix_scale.cpu().numpy(), 8, O.diag(42, IC), "f32")
    scores = O.index_scores(index_q.cpu().numpy(), index_w.cpu().numpy(), keys)
    tol = score_error_bound(index_q.cpu().numpy(), w_act(index_w.cpu().numpy(), "softplus"), keys,
                            extra_rel=96 * 2.0 ** -24)
    assert_topk_matches(idx.cpu().numpy(), scores, 256, tol)
    # ... and attention over the selected blocks vs the oracle on the same selection
    _close(out.view(B, H, D), _oracle_quant(pq, kv_codes, kv_scale, idx, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)


def test_config5_csa_decode_end_to_end(dev):
    # benchmark configuration cfg5: B=64, 65536 blocks (compression 4), 4-bit codes, N(0,1) with 2% outlier
    # channels x8, seed 4; indexer 4x64 softplus over all blocks, top-256 + window 128 + per-head sink
    # (serving.py:597-625).  Inputs as bench.py generates them.  Every row's selection against the
    # oracle's exact top-k (up to fp32 near-ties), attention against the oracle on that selection.
    from test_gpu_indexer import _oracle_rows_check

    B, H, D, S, W, IH, IC, seed = 64, 12, 128, 65536, 128, 4, 64, 4
    pq = PolarQuant(4)
    kv_codes, kv_scale = pq.encode(normal_with_outliers((B, S, D), seed, device=dev, trailing_dims=1))
    ix_codes, ix_scale = pq.encode(normal_with_outliers((B, S, IC), seed + 1000, device=dev, trailing_dims=1))
    q = normal((B, 1, H, D), seed + 1).to(dev)
    index_q = normal((B, IH, IC), seed + 2, dtype=torch.float32).to(dev)
    index_w = normal((B, IH), seed + 3, dtype=torch.float32).to(dev)
    win = normal((B, W, D), seed + 4).to(dev)
    sink = normal((H,), seed + 5, dtype=torch.float32).to(dev)
    sm = D ** -0.5
    print("cfg5 CSA decode, 64 rows", flush=True)
    out, idx = csa_decode(q, index_q, index_w, ix_codes, ix_scale, kv_codes, kv_scale, win, sink, sm, kv_quant=pq,
                          top_k=256)
    torch.cuda.synchronize()
    assert idx.shape == (B, 256) and out.shape == q.shape
    _oracle_rows_check(pq, ix_codes, ix_scale, index_q, index_w, idx.cpu().numpy(), 256, range(B))
    _close(out.view(B, H, D), _oracle_quant(pq, kv_codes, kv_scale, idx, q, win, sink, sm), QUANT_RTOL, QUANT_ATOL)


@pytest.fixture(params=["matrix", "generic"])
def attn_path(request):
    """Run a case on the matrix-core attention (default for head_dim 128) and on the generic one."""
    from aetherkv import _lib as L
    prev = L.lib().aekv_set_generic_kernels(1 if request.param == "generic" else 0)
    yield request.param
    L.lib().aekv_set_generic_kernels(prev)


@pytest.mark.parametrize("B,H,S,K,W,bits", [
    (3, 12, 100, 37, 0, 4),      # one partial tile, no window
    (2, 16, 300, None, 5, 8),    # every block (HCA), 3 tiles, 16 heads
    (2, 1, 50, 7, 130, 4),       # one head, window spills into a second tile
    (2, 12, 1200, None, 128, 4), # 11 tiles -> split over workgroups + combine
])
def test_quant_attention_head_dim_128_shapes(dev, attn_path, B, H, S, K, W, bits):
    D = 128
    pq, codes, scale, q, win, sink = _quant_inputs(dev, B, H, D, S, max(W, 1), bits, 60 + S % 89)
    win = win[:, :W].contiguous() if W else None
    sel = None
    if K is not None:
        g = torch.Generator().manual_seed(4)
        sel = torch.randint(-2, S + 2, (B, K), generator=g).to(dev)   # a few out-of-range entries
    sm = 0.11
    got = quant_sink_attention(q, codes, scale, sel, win, sink, sm, quant=pq)
    want = O.quant_attention(to_np_f32(q).reshape(B, H, D), codes.cpu().numpy(), scale.cpu().numpy(),
                             None if sel is None else sel.cpu().numpy(),
                             np.zeros((B, 0, D), np.float32) if win is None else to_np_f32(win), to_np_f32(sink),
                             O.diag(42, D), bits, sm)
    _close(got.view(B, H, D), want, QUANT_RTOL, QUANT_ATOL)
