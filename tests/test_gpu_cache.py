"""GPU tests of aetherkv.cache: the engine's quant helpers against the oracle, CodeRing appends against
a one-shot encode, and decode steps over rings against the same steps over compact tensors."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from aetherkv import PolarQuant
from aetherkv.cache import (CodeRing, DequantMemo, compressed_to_bf16_for_paging, csa_decode_ring, hca_decode_ring,
                            quant_append, read_compressed)
from aetherkv.decode import csa_decode, hca_decode
from conftest import bf16_bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [4, 8])
def test_quant_append_read_and_paging_match_oracle(dev, bits):
    B, D = 2, 128
    pq = PolarQuant(bits)
    g = torch.Generator(device=dev).manual_seed(3)
    data = scale = None
    xs = []
    for m in [1, 3, 1]:
        x = torch.randn(B, m, D, device=dev, generator=g).to(torch.bfloat16)
        data, scale = quant_append(pq, data, scale, x if m > 1 else x[:, 0])
        xs.append(x)
    allx = torch.cat(xs, dim=1)
    dg = O.diag(42, D)
    wc, ws = O.encode(bf16_bits(allx).reshape(-1, D), "bf16", bits, dg)
    assert data.shape[:2] == (B, 5) and scale.shape == (B, 5, 1)
    np.testing.assert_array_equal(data.cpu().numpy().reshape(wc.shape), wc)
    np.testing.assert_array_equal(scale.cpu().numpy().reshape(ws.shape), ws)
    memo = DequantMemo()
    r1 = read_compressed(pq, data, scale, torch.bfloat16, memo)
    assert read_compressed(pq, data, scale, torch.bfloat16, memo) is r1 and len(memo) == 1
    np.testing.assert_array_equal(bf16_bits(r1).reshape(-1, D), O.decode(wc, ws, bits, dg, "bf16"))
    page = compressed_to_bf16_for_paging(pq, data, scale, 1, 4, torch.bfloat16)
    np.testing.assert_array_equal(bf16_bits(page), bf16_bits(r1[:, 1:4]))
    assert compressed_to_bf16_for_paging(pq, data, scale, 2, 6, torch.bfloat16) is None


@pytest.mark.parametrize("bits", [4, 8])
def test_code_ring_matches_one_shot_encode(dev, bits):
    B, D = 3, 128
    pq = PolarQuant(bits)
    ring = CodeRing(pq, B, D, capacity=2, device=dev)
    g = torch.Generator(device=dev).manual_seed(5)
    xs = []
    for m in [1, 2, 1, 4, 1, 9]:
        x = torch.randn(B, m, D, device=dev, generator=g).to(torch.bfloat16)
        ring.append(x)
        xs.append(x)
    c, s = pq.encode(torch.cat(xs, dim=1))
    assert ring.n == 18 and ring.capacity == 32
    assert torch.equal(ring.data, c) and torch.equal(ring.scale, s)


def _csa_inputs(dev, B, n, bits, seed):
    H, D, W, IH, IC = 12, 128, 32, 4, 64
    g = torch.Generator(device=dev).manual_seed(seed)
    pq = PolarQuant(bits)
    kv_ring = CodeRing(pq, B, D, capacity=64, device=dev)
    ix_ring = CodeRing(pq, B, IC, capacity=64, device=dev)
    for m in [n // 3, n // 3, n - 2 * (n // 3)]:  # appends that grow the rings past n
        kv_ring.append(torch.randn(B, m, D, device=dev, generator=g).to(torch.bfloat16))
        ix_ring.append(torch.randn(B, m, IC, device=dev, generator=g).to(torch.bfloat16))
    q = torch.randn(B, 1, H, D, device=dev, generator=g).to(torch.bfloat16)
    iq = torch.randn(B, IH, IC, device=dev, generator=g)
    iw = torch.randn(B, IH, device=dev, generator=g)
    win = torch.randn(B, W, D, device=dev, generator=g).to(torch.bfloat16)
    sink = torch.randn(H, device=dev, generator=g)
    return pq, kv_ring, ix_ring, q, iq, iw, win, sink


@pytest.mark.parametrize("bits,n,top_k", [(4, 700, 256), (8, 500, 64), (4, 100, 256)])
def test_csa_decode_over_rings_matches_compact_tensors(dev, bits, n, top_k):
    B, D = 4, 128
    pq, kv_ring, ix_ring, q, iq, iw, win, sink = _csa_inputs(dev, B, n, bits, 17 + n)
    assert kv_ring.capacity > n  # the kernels read storage past the valid blocks
    out_r, idx_r = csa_decode_ring(q, iq, iw, ix_ring, kv_ring, win, sink, D ** -0.5, top_k=top_k)
    out_c, idx_c = csa_decode(q, iq, iw, ix_ring.data.contiguous(), ix_ring.scale.contiguous(),
                              kv_ring.data.contiguous(), kv_ring.scale.contiguous(), win, sink, D ** -0.5,
                              kv_quant=pq, top_k=top_k)
    assert idx_r.shape == (B, min(top_k, n))
    assert torch.equal(idx_r, idx_c)
    assert torch.equal(out_r, out_c)


def test_hca_decode_over_ring_matches_compact_tensors(dev):
    B, D, H, W, n = 3, 128, 12, 16, 1100  # 1116 sources: two splits
    g = torch.Generator(device=dev).manual_seed(23)
    pq = PolarQuant(4)
    ring = CodeRing(pq, B, D, capacity=512, device=dev)
    ring.append(torch.randn(B, 600, D, device=dev, generator=g).to(torch.bfloat16))
    ring.append(torch.randn(B, n - 600, D, device=dev, generator=g).to(torch.bfloat16))
    q = torch.randn(B, 1, H, D, device=dev, generator=g).to(torch.bfloat16)
    win = torch.randn(B, W, D, device=dev, generator=g).to(torch.bfloat16)
    sink = torch.randn(H, device=dev, generator=g)
    out_r = hca_decode_ring(q, ring, win, sink, D ** -0.5)
    out_c = hca_decode(q, ring.data.contiguous(), ring.scale.contiguous(), win, sink, D ** -0.5, kv_quant=pq)
    assert torch.equal(out_r, out_c)


@pytest.mark.parametrize("bits", [4, 8])
def test_paged_code_pages_round_trip_through_decode(dev, bits):
    # flush the leading blocks of single-sequence rings to code pages, materialise them back in front
    # of the resident blocks, and decode: identical to decoding the rings before paging
    from aetherkv.storage import flush_page, materialize_pages

    n, per_page = 700, 32
    pq, kv, ix, q, iq, iw, win, sink = _csa_inputs(dev, 1, n, bits, 31 + bits)
    out0, idx0 = csa_decode_ring(q, iq, iw, ix, kv, win, sink, 128 ** -0.5, top_k=256)
    pages = []
    while kv.n >= per_page:
        pages.append(flush_page({"layer1.csa": kv, "layer1.csa_index": ix},
                                {"layer1.csa": per_page, "layer1.csa_index": per_page}))
    assert len(pages) == n // per_page and kv.n == n % per_page
    kv2 = materialize_pages(pages, "layer1.csa", pq, 128, resident=kv)
    ix2 = materialize_pages(pages, "layer1.csa_index", pq, 64, resident=ix)
    assert kv2.n == n and ix2.n == n
    out1, idx1 = csa_decode_ring(q, iq, iw, ix2, kv2, win, sink, 128 ** -0.5, top_k=256)
    assert torch.equal(idx0, idx1)
    assert torch.equal(out0, out1)


@pytest.mark.parametrize("bits", [4, 8])
def test_code_pages_match_oracle(dev, bits):
    # The reference's paged allocator stores each flushed block as PolarQuant.decode of its code, in bf16
    # (serving.py:378-398, :857-905).  A code page stores the code itself: its rows must equal the
    # oracle's encode of the original blocks, their decode must equal the oracle's decode (the values the
    # reference's bf16 page holds), and a decode step over materialised pages must match the oracle's
    # exact top-k and its attention over that selection.
    from aetherkv.storage import flush_page, materialize_pages, unpack_rows
    from test_gpu_indexer import w_act
    from topk_check import assert_topk_matches, score_error_bound

    n, per_page, H, D, W, IH, IC = 700, 32, 12, 128, 32, 4, 64
    pq = PolarQuant(bits)
    g = torch.Generator().manual_seed(61 + bits)
    xk = torch.randn(1, n, D, generator=g).to(torch.bfloat16)
    xi = torch.randn(1, n, IC, generator=g).to(torch.bfloat16)
    kv, ix = CodeRing(pq, 1, D, capacity=64, device=dev), CodeRing(pq, 1, IC, capacity=64, device=dev)
    kv.append(xk.to(dev))
    ix.append(xi.to(dev))
    pages = []
    while kv.n >= per_page:
        pages.append(flush_page({"kv": kv, "ix": ix}, {"kv": per_page, "ix": per_page}))
    dg, dgi = O.diag(42, D), O.diag(42, IC)
    want_c, want_s = O.encode(bf16_bits(xk).reshape(n, D), "bf16", bits, dg)
    for i, p in enumerate(pages):
        c, s = unpack_rows(p["kv"], bits)
        rows = slice(i * per_page, (i + 1) * per_page)
        np.testing.assert_array_equal(c.cpu().numpy(), want_c[rows], err_msg=f"page {i} codes")
        np.testing.assert_array_equal(s.cpu().numpy(), want_s[rows], err_msg=f"page {i} scales")
        np.testing.assert_array_equal(bf16_bits(pq.decode(c, s)), O.decode(want_c[rows], want_s[rows], bits, dg, "bf16"),
                                      err_msg=f"page {i} decoded values")
    kv2 = materialize_pages(pages, "kv", pq, D, resident=kv)
    ix2 = materialize_pages(pages, "ix", pq, IC, resident=ix)
    gq = torch.Generator().manual_seed(71 + bits)
    q = torch.randn(1, 1, H, D, generator=gq).to(torch.bfloat16).to(dev)
    iq = torch.randn(1, IH, IC, generator=gq).to(dev)
    iw = torch.randn(1, IH, generator=gq).to(dev)
    win = torch.randn(1, W, D, generator=gq).to(torch.bfloat16).to(dev)
    sink = torch.randn(H, generator=gq).to(dev)
    out, idx = csa_decode_ring(q, iq, iw, ix2, kv2, win, sink, D ** -0.5, top_k=256)
    # oracle: keys from the ORIGINAL blocks' codes
    ic, is_ = O.encode(bf16_bits(xi).reshape(n, IC), "bf16", bits, dgi)
    keys = O.decode(ic, is_, bits, dgi, "f32").reshape(1, n, IC)
    qn, wn = iq.cpu().numpy(), iw.cpu().numpy()
    scores = O.index_scores(qn, wn, keys)
    tol = score_error_bound(qn, w_act(wn, "softplus"), keys, extra_rel=96 * 2.0 ** -24)
    assert_topk_matches(idx.cpu().numpy(), scores, 256, tol)
    want = O.quant_attention(q.float().cpu().numpy().reshape(1, H, D), want_c.reshape(1, n, -1),
                             want_s.reshape(1, n), idx.cpu().numpy(), win.float().cpu().numpy(),
                             sink.cpu().numpy(), dg, bits, D ** -0.5)
    np.testing.assert_allclose(out.float().cpu().numpy().reshape(1, H, D), want, rtol=1e-2, atol=2e-3)
