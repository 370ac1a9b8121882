"""HIP-graph capture of the decode step (indexer + attention, CSA and HCA).

The kernels clear memory with fill kernels (no hipMemsetAsync), take no host synchronisation and
allocate nothing when given workspaces and outputs, so a serving loop can capture them.  Every
replay is checked against the eager result of the same inputs, with eager work and input changes
between replays.
"""
from __future__ import annotations

import pytest
import torch

from aetherkv import PolarQuant
from aetherkv.decode import attention_workspace, csa_indexer_topk_quant, indexer_workspace, quant_sink_attention

pytestmark = pytest.mark.gpu


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


@pytest.mark.parametrize("bits", [4, 8])
def test_csa_step_graph_replays_match_eager(dev, bits):
    B, S, H, D, W, IH, IC, k = 4, 3000, 12, 128, 32, 4, 64, 64
    gen = torch.Generator(device=dev).manual_seed(7 + bits)
    pq = PolarQuant(bits)
    kv_codes, kv_scale = pq.encode(torch.randn(B, S, D, device=dev, generator=gen).to(torch.bfloat16))
    ix_codes, ix_scale = pq.encode(torch.randn(B, S, IC, device=dev, generator=gen).to(torch.bfloat16))
    # static inputs of the captured step, changed in place between replays
    iq = torch.randn(B, IH, IC, device=dev, generator=gen)
    iw = torch.randn(B, IH, device=dev, generator=gen)
    q = torch.randn(B, 1, H, D, device=dev, generator=gen).to(torch.bfloat16)
    win = torch.randn(B, W, D, device=dev, generator=gen).to(torch.bfloat16)
    sink = torch.randn(H, device=dev, generator=gen)
    ws_i, ws_a = indexer_workspace(B, S, k, dev), attention_workspace(B, H, D, k, W, dev)
    idx_g = torch.empty(B, k, dtype=torch.int64, device=dev)
    out_g = torch.empty(B, H, D, dtype=torch.bfloat16, device=dev)

    def step(idx, out, wi, wa):
        csa_indexer_topk_quant(iq, iw, ix_codes, ix_scale, k, quant=pq, workspace=wi, out=idx)
        quant_sink_attention(q, kv_codes, kv_scale, idx, win, sink, D ** -0.5, quant=pq, workspace=wa, out=out)

    g = _capture(lambda: step(idx_g, out_g, ws_i, ws_a))
    for rep in range(3):
        if rep > 0:  # new inputs in the captured tensors
            iq.copy_(torch.randn(B, IH, IC, device=dev, generator=gen))
            q.copy_(torch.randn(B, 1, H, D, device=dev, generator=gen).to(torch.bfloat16))
        # eager reference with its own workspaces and outputs, then a synchronisation
        idx_e = torch.empty_like(idx_g)
        out_e = torch.empty_like(out_g)
        step(idx_e, out_e, indexer_workspace(B, S, k, dev), attention_workspace(B, H, D, k, W, dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx_g, idx_e), f"replay {rep}: top-k differs from eager"
        assert torch.equal(out_g, out_e), f"replay {rep}: attention differs from eager"


def test_hca_step_graph_replays_match_eager(dev):
    B, S, H, D, W = 3, 1500, 12, 128, 16  # 1516 sources: two splits and the combine kernel
    gen = torch.Generator(device=dev).manual_seed(11)
    pq = PolarQuant(4)
    codes, scale = pq.encode(torch.randn(B, S, D, device=dev, generator=gen).to(torch.bfloat16))
    q = torch.randn(B, 1, H, D, device=dev, generator=gen).to(torch.bfloat16)
    win = torch.randn(B, W, D, device=dev, generator=gen).to(torch.bfloat16)
    sink = torch.randn(H, device=dev, generator=gen)
    ws = attention_workspace(B, H, D, S, W, dev)
    out_g = torch.empty(B, H, D, dtype=torch.bfloat16, device=dev)
    g = _capture(lambda: quant_sink_attention(q, codes, scale, None, win, sink, D ** -0.5, quant=pq, workspace=ws,
                                              out=out_g))
    for rep in range(3):
        if rep > 0:
            q.copy_(torch.randn(B, 1, H, D, device=dev, generator=gen).to(torch.bfloat16))
        out_e = quant_sink_attention(q, codes, scale, None, win, sink, D ** -0.5, quant=pq)  # [B, 1, H, D]
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e.view(B, H, D)), f"replay {rep}: HCA attention differs from eager"
