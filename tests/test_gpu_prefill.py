"""GPU tests of chunked prefill through the quantised reader (aetherkv.prefill).

Each target of a chunk is checked against the oracle's decode-step attention on that target's own
sources (its visible blocks or its indexer selection, and its window slice; modeling.py:316-325 /
:521-539), within the bf16 tolerance of the quantised attention tests.  CSA targets are also
checked bit for bit against the decode entry point called once per target on the same sources
(the per-target rows reuse the decode kernel), and the multi-target indexer bit for bit against
the single-target indexer per target and its selection against the oracle's exact top-k up to
fp32 near-ties.  HCA prefill runs a different kernel (blocks decoded once, then a flash-style
pass shared by many targets), so its bar is the oracle tolerance and closeness to the decode
launches within the same tolerance.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
from aetherkv import PolarQuant
from aetherkv.decode import csa_indexer_topk_quant, quant_sink_attention
from aetherkv.prefill import (csa_prefill, csa_prefill_indexer_topk_quant, hca_prefill, prefill_sources,
                              quant_prefill_attention)
from aetherkv.synthetic import normal
from conftest import to_np_f32
from topk_check import assert_topk_matches, score_error_bound

pytestmark = pytest.mark.gpu

QUANT_RTOL, QUANT_ATOL = 1e-2, 2e-3  # bf16 output, as the decode-step quantised attention tests


def _inputs(dev, B, T, H, S, Wt, bits, seed, D=128):
    pq = PolarQuant(bits)
    codes, scale = pq.encode(normal((B, S, D), seed).to(dev))
    q = normal((B, T, H, D), seed + 1).to(dev)
    win = normal((B, Wt, D), seed + 2).to(dev)
    sink = normal((H,), seed + 3, dtype=torch.float32).to(dev)
    return pq, codes, scale, q, win, sink


@pytest.fixture(params=[64, 96])
def flash_rows(request):
    """Run an HCA case on each workgroup shape of the flash kernel (64 rows / 4 waves, 96 rows / 12
    waves); the default picks one per launch."""
    from aetherkv import _lib as L
    prev = L.lib().aekv_set_flash_rows(request.param)
    yield request.param
    L.lib().aekv_set_flash_rows(prev)


def _oracle_target(pq, codes, scale, sel_np, q_t, win_t, sink, sm):
    B, H, D = q_t.shape
    return O.quant_attention(to_np_f32(q_t), codes.cpu().numpy(), scale.cpu().numpy(), sel_np, to_np_f32(win_t),
                             to_np_f32(sink), O.diag(42, D), pq.bits, sm)


@pytest.mark.parametrize("bits,B,T,H,start,M,W,nb,S", [
    (4, 2, 40, 12, 100, 8, 16, 17, 24),     # capacity past the emitted blocks; targets cross block edges
    (8, 3, 33, 16, 0, 4, 8, 8, 8),          # first chunk: the early targets see no block
    (4, 2, 6, 12, 9000, 8, 128, 1130, 1200),  # ~1250 sources per target
    (4, 2, 200, 12, 6300, 128, 128, 60, 64),  # the model's HCA shape: a block edge inside the chunk
    (8, 1, 70, 5, 37, 4, 20, 30, 40),       # rows per workgroup not a multiple of the head count
])
def test_hca_prefill_matches_oracle_and_decode(dev, flash_rows, bits, B, T, H, start, M, W, nb, S):
    Wt = W - 1 + T
    pq, codes, scale, q, win, sink = _inputs(dev, B, T, H, S, Wt, bits, 7 + T)
    sm = 128 ** -0.5
    print(f"hca prefill rows={flash_rows} bits={bits} B={B} T={T} H={H} start={start} nb={nb}", flush=True)
    out = hca_prefill(q, codes, scale, win, sink, sm, kv_quant=pq, start=start, n_blocks=nb, compression=M,
                      sliding_window=W)
    torch.cuda.synchronize()
    assert out.shape == (B, T, H, 128) and out.dtype == torch.bfloat16
    vis, ws, wl = prefill_sources(T, start, nb, compression=M, sliding_window=W, window_base=start + T - Wt,
                                  window_len=Wt)
    for t in range(T):
        g, s0, n = int(vis[t]), int(ws[t]), int(wl[t])
        win_t = win[:, s0:s0 + n].contiguous()
        sel = np.tile(np.arange(g, dtype=np.int64), (B, 1))
        want = _oracle_target(pq, codes, scale, sel, q[:, t], win_t, sink, sm)
        np.testing.assert_allclose(to_np_f32(out[:, t]), want, rtol=QUANT_RTOL, atol=QUANT_ATOL,
                                   err_msg=f"target {t}")
        # the decode entry point on the same sources (blocks 0..g-1 in order, the same window slice)
        dec = quant_sink_attention(q[:, t], codes[:, :g].contiguous(), scale[:, :g].contiguous(), None, win_t, sink,
                                   sm, quant=pq)
        np.testing.assert_allclose(to_np_f32(out[:, t]), to_np_f32(dec), rtol=QUANT_RTOL, atol=QUANT_ATOL,
                                   err_msg=f"target {t} vs the decode launch")


@pytest.mark.parametrize("bits", [4, 8])
def test_csa_prefill_matches_oracle_and_decode(dev, bits):
    B, T, H, IH, IC, M, W, top_k = 2, 48, 12, 4, 64, 4, 16, 5
    start, nb = 20, 17  # positions 20..67: 5..16 visible blocks, more than top_k from position 24 on
    Wt = W - 1 + T
    pq, codes, scale, q, win, sink = _inputs(dev, B, T, H, 24, Wt, bits, 50 + bits)
    ix_codes, ix_scale = pq.encode(normal((B, 24, IC), 60 + bits).to(dev))
    index_q = normal((B, T, IH, IC), 61, dtype=torch.float32).to(dev)
    index_w = normal((B, T, IH), 62, dtype=torch.float32).to(dev)
    sm = 128 ** -0.5
    print(f"csa prefill bits={bits}", flush=True)
    out, idx = csa_prefill(q, index_q, index_w, ix_codes, ix_scale, codes, scale, win, sink, sm, kv_quant=pq,
                           start=start, n_blocks=nb, compression=M, sliding_window=W, top_k=top_k)
    torch.cuda.synchronize()
    assert idx.shape == (B, T, top_k) and out.shape == (B, T, H, 128)
    vis, ws, wl = prefill_sources(T, start, nb, compression=M, sliding_window=W, window_base=start + T - Wt,
                                  window_len=Wt)
    keys = O.decode(ix_codes.cpu().numpy(), ix_scale.cpu().numpy(), bits, O.diag(42, IC), "f32")
    for t in range(T):
        g, s0, n = int(vis[t]), int(ws[t]), int(wl[t])
        k_eff = min(top_k, g)
        # the target's selection: one indexer row per target vs the single-target indexer
        one = csa_indexer_topk_quant(index_q[:, t], index_w[:, t], ix_codes, ix_scale, top_k, quant=pq,
                                     valid=torch.full((B,), g, dtype=torch.int32, device=dev))
        assert torch.equal(idx[:, t], one), f"target {t}: selection differs from the single-target indexer"
        qn, wn = index_q[:, t].cpu().numpy(), index_w[:, t].cpu().numpy()
        scores = O.index_scores(qn, wn, keys, valid=np.full(B, g, np.int32))
        wa = np.log1p(np.exp(wn.astype(np.float64)))
        tol = score_error_bound(qn, wa, keys, extra_rel=16 * math.log2(IC) * 2.0 ** -24)
        assert_topk_matches(idx[:, t].cpu().numpy(), scores, top_k, tol, np.full(B, g))
        # attention over the selected blocks and the window slice
        sel = idx[:, t, :k_eff].contiguous()
        win_t = win[:, s0:s0 + n].contiguous()
        want = _oracle_target(pq, codes, scale, sel.cpu().numpy(), q[:, t], win_t, sink, sm)
        np.testing.assert_allclose(to_np_f32(out[:, t]), want, rtol=QUANT_RTOL, atol=QUANT_ATOL,
                                   err_msg=f"target {t}")
        dec = quant_sink_attention(q[:, t], codes, scale, sel, win_t, sink, sm, quant=pq)
        assert torch.equal(out[:, t], dec), f"target {t} differs from the decode launch"


@pytest.mark.parametrize("bits,IH,IC", [(4, 4, 64), (8, 8, 128), (4, 6, 64)])
def test_multi_target_indexer_ragged_valid(dev, bits, IH, IC):
    # per-(row, target) visible counts, including 0 and counts below k; the targets go through the
    # score kernel 4 per key group (IH 5..8: two 4-head row blocks), the reference through the
    # single-target kernel
    B, T, S, k = 3, 7, 3000, 64
    pq = PolarQuant(bits)
    codes, scale = pq.encode(normal((B, S, IC), 71).to(dev))
    index_q = normal((B, T, IH, IC), 72, dtype=torch.float32).to(dev)
    index_w = normal((B, T, IH), 73, dtype=torch.float32).to(dev)
    valid = torch.tensor([[0, 1, 63, 64, 65, 2999, 3000], [5, 5, 5, 5, 5, 5, 5], [3000, 0, 1000, 17, 64, 1, 2]],
                         dtype=torch.int32)
    print(f"multi-target indexer ragged bits={bits} IH={IH} IC={IC}", flush=True)
    idx, sc = csa_prefill_indexer_topk_quant(index_q, index_w, codes, scale, k, quant=pq, valid=valid,
                                             return_scores=True)
    torch.cuda.synchronize()
    for t in range(T):
        one, sc1 = csa_indexer_topk_quant(index_q[:, t], index_w[:, t], codes, scale, k, quant=pq,
                                          valid=valid[:, t].to(dev), return_scores=True)
        assert torch.equal(idx[:, t], one), f"target {t}"
        assert torch.equal(sc[:, t], sc1), f"target {t} scores"
    assert bool((idx[0, 0] == -1).all()) and int((idx[1] >= 0).sum(-1).max()) == 5
    # and against the oracle's exact top-k (up to fp32 near-ties)
    keys = O.decode(codes.cpu().numpy(), scale.cpu().numpy(), bits, O.diag(42, IC), "f32")
    for t in range(T):
        qn, wn = index_q[:, t].cpu().numpy(), index_w[:, t].cpu().numpy()
        vt = valid[:, t].numpy()
        scores = O.index_scores(qn, wn, keys, valid=vt)
        wa = np.log1p(np.exp(wn.astype(np.float64)))
        tol = score_error_bound(qn, wa, keys, extra_rel=16 * math.log2(IC) * 2.0 ** -24)
        assert_topk_matches(idx[:, t].cpu().numpy(), scores, k, tol, vt)


def test_multi_target_indexer_many_rows(dev):
    # >= 1024 rows with k <= 512 select through the 512-thread kernel: sampled targets against the
    # single-target indexer (1024-thread kernel) bit for bit and against the oracle's exact top-k
    B, T, S, IH, IC, k = 2, 512, 2500, 4, 64, 256
    pq = PolarQuant(8)
    codes, scale = pq.encode(normal((B, S, IC), 81).to(dev))
    index_q = normal((B, T, IH, IC), 82, dtype=torch.float32).to(dev)
    index_w = normal((B, T, IH), 83, dtype=torch.float32).to(dev)
    valid = torch.randint(0, S + 1, (B, T), generator=torch.Generator().manual_seed(84), dtype=torch.int32)
    valid[0, :8] = torch.tensor([0, 1, 255, 256, 257, S, S - 1, 511], dtype=torch.int32)
    print("multi-target indexer, 1024 rows", flush=True)
    idx = csa_prefill_indexer_topk_quant(index_q, index_w, codes, scale, k, quant=pq, valid=valid)
    torch.cuda.synchronize()
    keys = O.decode(codes.cpu().numpy(), scale.cpu().numpy(), 8, O.diag(42, IC), "f32")
    for t in list(range(8)) + list(range(9, T, 37)):
        one = csa_indexer_topk_quant(index_q[:, t], index_w[:, t], codes, scale, k, quant=pq,
                                     valid=valid[:, t].to(dev))
        assert torch.equal(idx[:, t], one), f"target {t}"
        qn, wn = index_q[:, t].cpu().numpy(), index_w[:, t].cpu().numpy()
        vt = valid[:, t].numpy()
        scores = O.index_scores(qn, wn, keys, valid=vt)
        tol = score_error_bound(qn, np.log1p(np.exp(wn.astype(np.float64))), keys,
                                extra_rel=16 * math.log2(IC) * 2.0 ** -24)
        assert_topk_matches(idx[:, t].cpu().numpy(), scores, k, tol, vt)


def test_hca_prefill_window_only(dev, flash_rows):
    # no compressed block yet (an empty cache): every target attends its window slice and the sink
    B, T, H, W, bits = 2, 40, 12, 16, 4
    Wt = W - 1 + T
    pq = PolarQuant(bits)
    codes = torch.zeros((B, 0, 64), dtype=torch.uint8, device=dev)
    scale = torch.zeros((B, 0), dtype=torch.float32, device=dev)
    q = normal((B, T, H, 128), 401).to(dev)
    win = normal((B, Wt, 128), 402).to(dev)
    sink = normal((H,), 403, dtype=torch.float32).to(dev)
    sm = 128 ** -0.5
    print(f"hca prefill window only rows={flash_rows}", flush=True)
    out = hca_prefill(q, codes, scale, win, sink, sm, kv_quant=pq, start=0, n_blocks=0, compression=128,
                      sliding_window=W)
    torch.cuda.synchronize()
    vis, ws, wl = prefill_sources(T, 0, 0, compression=128, sliding_window=W, window_base=T - Wt, window_len=Wt)
    assert int(vis.max()) == 0
    for t in range(T):
        s0, n = int(ws[t]), int(wl[t])
        want = _oracle_target(pq, codes, scale, np.zeros((B, 0), dtype=np.int64), q[:, t],
                              win[:, s0:s0 + n].contiguous(), sink, sm)
        np.testing.assert_allclose(to_np_f32(out[:, t]), want, rtol=QUANT_RTOL, atol=QUANT_ATOL, err_msg=f"target {t}")


def test_hca_prefill_chunk_both_workgroup_shapes(dev):
    # The bench's HCA chunk (B=8, T=256 targets at the end of a 262144-token prompt, 2048 4-bit
    # blocks, H=12, W=128): 24576 (target, head) rows, where the default launch takes the 96-row
    # shape on a 256-CU device.  Both shapes against the oracle on sampled targets, against each
    # other within the tolerance, and the default bit for bit against the shape it picked.
    from aetherkv import _lib as L
    B, T, H, S, M, W, bits = 8, 256, 12, 2048, 128, 128, 4
    start, Wt = S * M - T, W - 1 + T
    pq, codes, scale, q, win, sink = _inputs(dev, B, T, H, S, Wt, bits, 501)
    sm = 128 ** -0.5
    vis, ws, wl = prefill_sources(T, start, S, compression=M, sliding_window=W, window_base=start - (W - 1),
                                  window_len=Wt)
    args = dict(quant=pq, visible=vis.to(dev), win_start=ws.to(dev), win_len=wl.to(dev))
    outs = {}
    for rows in (0, 64, 96):
        print(f"hca prefill chunk rows={rows}", flush=True)
        prev = L.lib().aekv_set_flash_rows(rows)
        try:
            outs[rows] = quant_prefill_attention(q, codes, scale, None, win, sink, sm, **args)
            torch.cuda.synchronize()
        finally:
            L.lib().aekv_set_flash_rows(prev)
    assert torch.equal(outs[0], outs[64]) or torch.equal(outs[0], outs[96])
    np.testing.assert_allclose(to_np_f32(outs[64]), to_np_f32(outs[96]), rtol=QUANT_RTOL, atol=QUANT_ATOL)
    for t in (0, 1, 95, 96, 200, T - 1):
        g, s0, n = int(vis[t]), int(ws[t]), int(wl[t])
        for b in (0, B - 1):
            sel = np.arange(g, dtype=np.int64)[None]
            want = _oracle_target(pq, codes[b:b + 1], scale[b:b + 1], sel, q[b:b + 1, t],
                                  win[b:b + 1, s0:s0 + n].contiguous(), sink, sm)
            for rows in (64, 96):
                np.testing.assert_allclose(to_np_f32(outs[rows][b, t])[None], want, rtol=QUANT_RTOL,
                                           atol=QUANT_ATOL, err_msg=f"rows {rows} target {t} sequence {b}")


def test_prefill_attention_defaults_and_empty_targets(dev):
    # visible / window slices omitted: every target sees all n_sel blocks and the whole window; a
    # target with no source at all gets zeros (serving.py:451-452)
    B, T, H, S, Wt = 2, 3, 4, 40, 6
    pq, codes, scale, q, win, sink = _inputs(dev, B, T, H, S, Wt, 8, 91)
    sel = torch.randint(0, S, (B, T, 9), generator=torch.Generator().manual_seed(1)).to(dev)
    sel[0, 1, :4] = -1
    sm = 0.2
    print("prefill defaults and empty targets", flush=True)
    out = quant_prefill_attention(q, codes, scale, sel, win, sink, sm, quant=pq)
    for t in range(T):
        dec = quant_sink_attention(q[:, t], codes, scale, sel[:, t].contiguous(), win, sink, sm, quant=pq)
        assert torch.equal(out[:, t], dec), f"target {t}"
    zeros = torch.zeros(T, dtype=torch.int32)
    out = quant_prefill_attention(q, codes, scale, sel, win, sink, sm, quant=pq, visible=zeros, win_len=zeros)
    torch.cuda.synchronize()
    assert not bool(out.float().abs().sum())


def test_prefill_rejects_unsupported_shapes(dev):
    pq = PolarQuant(4)
    q = torch.zeros(1, 2, 17, 128, dtype=torch.bfloat16, device=dev)  # 17 heads: above the matrix-core limit
    codes = torch.zeros(1, 3, 64, dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="16 supported"):
        quant_prefill_attention(q, codes, torch.ones(1, 3, device=dev), None, None, torch.zeros(17, device=dev),
                                0.1, quant=pq)


@pytest.mark.parametrize("bits", [4, 8])
def test_prefill_attention_many_rows(dev, bits):
    # >= 1024 rows: the attention runs its 4-wave workgroup instance.  Ragged per-target selections
    # (some entries out of range) and window slices; sampled targets against the oracle and against
    # the decode entry point on the same sources (the 8-wave instance), both within the tolerance.
    B, T, H, S, K, Wt = 2, 512, 12, 3000, 256, 160
    pq, codes, scale, q, win, sink = _inputs(dev, B, T, H, S, Wt, bits, 120 + bits)
    g = torch.Generator().manual_seed(121 + bits)
    sel = torch.randint(-3, S + 3, (B, T, K), generator=g)
    visible = torch.randint(0, K + 1, (B, T), generator=g, dtype=torch.int32)
    visible[0, :4] = torch.tensor([0, 1, K, K - 1], dtype=torch.int32)
    win_start = torch.randint(0, Wt, (B, T), generator=g, dtype=torch.int32)
    win_len = torch.randint(0, 129, (B, T), generator=g, dtype=torch.int32)
    win_len = torch.minimum(win_len, Wt - win_start)
    win_len[1, :3] = 0
    sm = 128 ** -0.5
    print(f"prefill attention 1024 rows bits={bits}", flush=True)
    out = quant_prefill_attention(q, codes, scale, sel.to(dev), win, sink, sm, quant=pq, visible=visible.to(dev),
                                  win_start=win_start.to(dev), win_len=win_len.to(dev))
    torch.cuda.synchronize()
    for t in list(range(6)) + list(range(7, T, 41)):
        for b in range(B):
            g_, s0, n = int(visible[b, t]), int(win_start[b, t]), int(win_len[b, t])
            st = sel[b:b + 1, t, :g_].contiguous()
            win_t = win[b:b + 1, s0:s0 + n].contiguous()
            want = _oracle_target(pq, codes[b:b + 1], scale[b:b + 1], st.numpy(), q[b:b + 1, t], win_t, sink, sm)
            np.testing.assert_allclose(to_np_f32(out[b, t])[None], want, rtol=QUANT_RTOL, atol=QUANT_ATOL,
                                       err_msg=f"target {t} row {b}")
            dec = quant_sink_attention(q[b:b + 1, t], codes[b:b + 1].contiguous(), scale[b:b + 1].contiguous(),
                                       st.to(dev), win_t if n else None, sink, sm, quant=pq)
            np.testing.assert_allclose(to_np_f32(out[b, t]), to_np_f32(dec[0]), rtol=QUANT_RTOL, atol=QUANT_ATOL,
                                       err_msg=f"target {t} row {b} vs the decode launch")
