"""GPU tests of the one-call CSA decode step (aekv_csa_decode_quant, aetherkv.decode.csa_decode_step).

Where its fused kernel applies, the selection and the attention of a row run in one workgroup; the
results must be those of the two separate entry points (aekv_csa_indexer_topk_quant, then
aekv_quant_sink_attention over its selection): the selection and its scores bit for bit, and the
attention within the attention tolerance (the fused kernel attends the window first, while the
select runs, so its sources are summed in another order), and within the tolerance of the oracle.
Outside the fused kernel's limits the entry point runs the two separate entry points itself, with
identical results.  The oracle checks of the same step are in
test_gpu_attention.py (cfg3, cfg5) and test_gpu_cache.py.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from aetherkv import PolarQuant
from aetherkv.decode import csa_decode_step, csa_indexer_topk_quant, quant_sink_attention
from aetherkv.synthetic import normal, normal_with_outliers
from conftest import to_np_f32

pytestmark = pytest.mark.gpu


def _inputs(dev, B, S, H, IH, IC, W, kv_bits, ix_bits, seed, outliers=False):
    gen = (lambda shape, s: normal_with_outliers(shape, s, device=dev, trailing_dims=1)) if outliers else \
        (lambda shape, s: normal(shape, s, device=dev))
    kvq, ixq = PolarQuant(kv_bits), PolarQuant(ix_bits)
    kv_codes, kv_scale = kvq.encode(gen((B, S, 128), seed))
    ix_codes, ix_scale = ixq.encode(gen((B, S, IC), seed + 1))
    return dict(kvq=kvq, ixq=ixq, kv_codes=kv_codes, kv_scale=kv_scale, ix_codes=ix_codes, ix_scale=ix_scale,
                q=normal((B, 1, H, 128), seed + 2, device=dev),
                iq=normal((B, IH, IC), seed + 3, dtype=torch.float32, device=dev),
                iw=normal((B, IH), seed + 4, dtype=torch.float32, device=dev),
                win=normal((B, W, 128), seed + 5, device=dev) if W else None,
                sink=normal((H,), seed + 6, dtype=torch.float32, device=dev))


@pytest.mark.parametrize("B,S,H,IH,IC,W,k,kv_bits,ix_bits,mode,valid", [
    (8, 16384, 12, 4, 64, 128, 256, 8, 8, "softplus", None),                    # cfg3
    (16, 65536, 12, 4, 64, 128, 256, 4, 4, "softplus", None),                   # cfg5's shape, 16 rows
    (6, 5000, 12, 4, 64, 128, 256, 4, 4, "softplus", [5000, 0, 1, 255, 256, 3000]),   # ragged, padding
    (4, 3000, 16, 4, 64, 0, 64, 8, 4, "raw", [3000, 70, 64, 2]),                # no window, mixed widths
    (3, 4000, 1, 8, 128, 37, 100, 4, 8, "relu_w", None),                        # one head, IC 128, 8 index heads
    (2, 20000, 12, 16, 64, 128, 384, 4, 4, "softplus", None),                   # 16 index heads, 512 sources
    (3, 9000, 12, 4, 64, 5, 256, 8, 8, "softplus", [9000, 0, 300]),             # window of 5, an empty row
    (2, 70000, 12, 4, 64, 127, 512, 4, 4, "softplus", None),                    # 16 selected groups, W = 127
])
def test_decode_step_equals_separate_entry_points(dev, B, S, H, IH, IC, W, k, kv_bits, ix_bits, mode, valid):
    x = _inputs(dev, B, S, H, IH, IC, W, kv_bits, ix_bits, 200 + S % 97, outliers=kv_bits == 4)
    vd = None if valid is None else torch.tensor(valid, dtype=torch.int32, device=dev)
    sm = 128 ** -0.5
    print(f"decode step B={B} S={S} H={H} IH={IH} IC={IC} W={W} k={k} bits={kv_bits}/{ix_bits} {mode}", flush=True)
    out, idx, sc = csa_decode_step(x["q"], x["iq"], x["iw"], x["ix_codes"], x["ix_scale"], x["kv_codes"], x["kv_scale"],
                                   x["win"], x["sink"], sm, k, kv_quant=x["kvq"], index_quant=x["ixq"], valid=vd,
                                   mode=mode, return_scores=True)
    idx1, sc1 = csa_indexer_topk_quant(x["iq"], x["iw"], x["ix_codes"], x["ix_scale"], k, quant=x["ixq"], valid=vd,
                                       mode=mode, return_scores=True)
    out1 = quant_sink_attention(x["q"], x["kv_codes"], x["kv_scale"], idx1, x["win"], x["sink"], sm, quant=x["kvq"])
    torch.cuda.synchronize()
    assert torch.equal(idx, idx1)
    assert torch.equal(sc, sc1)
    np.testing.assert_allclose(to_np_f32(out), to_np_f32(out1), rtol=1e-2, atol=2e-3)
    # and the attention against the oracle on the returned selection
    want = O.quant_attention(to_np_f32(x["q"]).reshape(B, H, 128), x["kv_codes"].cpu().numpy(),
                             x["kv_scale"].cpu().numpy(), idx.cpu().numpy(),
                             np.zeros((B, 0, 128), np.float32) if x["win"] is None else to_np_f32(x["win"]),
                             to_np_f32(x["sink"]), O.diag(42, 128), kv_bits, sm)
    np.testing.assert_allclose(to_np_f32(out).reshape(B, H, 128), want, rtol=1e-2, atol=2e-3)


@pytest.mark.parametrize("ix_bits,n_special,S", [(4, 300, 20000), (8, 300, 20000), (4, 100, 20000), (8, 100, 20000),
                                                  (4, 100, 65536), (4, "spread", 20000), (4, "spread", 65536),
                                                  # rows of at most 16384 keys
                                                  (8, 300, 16384), (4, 100, 16384), (4, "spread", 12000)])
def test_decode_step_exact_ties(dev, ix_bits, n_special, S):
    # Every index key is the same code row (equal scores).  With an integer n_special, that many
    # keys get twice the scale: with 100 the k-th key is one of all the other, equal keys, so the
    # fused select's candidates overflow its LDS list and the radix levels run over every stored
    # key of the row (at S = 65536 every slot qualifies, more than its slot list holds).  "spread":
    # 300 keys get scales 2^(1 + 12 i / 300) times the common one, which puts the k-th largest slot
    # maximum ~10 binades below the row's largest, past the select's per-wave threshold search.
    B, H, IH, IC, W, k = 2, 12, 4, 64, 32, 256
    kvq, ixq = PolarQuant(4), PolarQuant(ix_bits)
    kv_codes, kv_scale = kvq.encode(normal((B, S, 128), 31, device=dev))
    row = normal((1, 1, IC), 5, dtype=torch.bfloat16)
    ix_codes, ix_scale = ixq.encode(row.expand(B, S, IC).contiguous().to(dev))
    iq = normal((B, IH, IC), 6, dtype=torch.float32)
    keyf = ixq.decode(ix_codes[:1, :1], ix_scale[:1, :1], out_dtype=torch.float32).cpu()[0, 0]
    iq = torch.where((iq @ keyf)[..., None] < 0, -iq, iq).to(dev)   # positive dots: nonzero scores
    iw = torch.ones(B, IH, device=dev)
    g = torch.Generator().manual_seed(9)
    ix_scale = ix_scale.clone()
    for b in range(B):
        if n_special == "spread":
            mult = torch.tensor([2.0 ** (1 + 12 * i / 300) for i in range(300)], dtype=torch.float32, device=dev)
            ix_scale[b, torch.randperm(S, generator=g)[:300].to(dev)] *= mult[:, None]
        else:
            ix_scale[b, torch.randperm(S, generator=g)[:n_special].to(dev)] *= 2
    q = normal((B, 1, H, 128), 7, device=dev)
    win = normal((B, W, 128), 8, device=dev)
    sink = normal((H,), 9, dtype=torch.float32, device=dev)
    sm = 128 ** -0.5
    print(f"decode step exact ties bits={ix_bits} specials={n_special} S={S}", flush=True)
    out, idx, sc = csa_decode_step(q, iq, iw, ix_codes, ix_scale, kv_codes, kv_scale, win, sink, sm, k, kv_quant=kvq,
                                   index_quant=ixq, return_scores=True)
    idx1, sc1 = csa_indexer_topk_quant(iq, iw, ix_codes, ix_scale, k, quant=ixq, return_scores=True)
    out1 = quant_sink_attention(q, kv_codes, kv_scale, idx1, win, sink, sm, quant=kvq)
    torch.cuda.synchronize()
    assert torch.equal(idx, idx1) and torch.equal(sc, sc1)
    np.testing.assert_allclose(to_np_f32(out), to_np_f32(out1), rtol=1e-2, atol=2e-3)


@pytest.mark.parametrize("k,W", [(600, 128), (512, 600)])
def test_decode_step_outside_the_fused_limits(dev, k, W):
    # k > 512 or k + W > 1024: the entry point runs the indexer and the attention entry points in turn
    B, S, H = 3, 9000, 12
    x = _inputs(dev, B, S, H, 4, 64, W, 8, 8, 77)
    sm = 0.09
    out, idx = csa_decode_step(x["q"], x["iq"], x["iw"], x["ix_codes"], x["ix_scale"], x["kv_codes"], x["kv_scale"],
                               x["win"], x["sink"], sm, k, kv_quant=x["kvq"], index_quant=x["ixq"])
    idx1 = csa_indexer_topk_quant(x["iq"], x["iw"], x["ix_codes"], x["ix_scale"], k, quant=x["ixq"])
    out1 = quant_sink_attention(x["q"], x["kv_codes"], x["kv_scale"], idx1, x["win"], x["sink"], sm, quant=x["kvq"])
    torch.cuda.synchronize()
    assert torch.equal(idx, idx1) and torch.equal(out, out1)


def test_decode_step_replays_in_a_graph(dev):
    # captured once, replayed three times with the inputs changed in place between replays: every
    # replay equals the eager step
    B, S, H, W, k = 8, 16384, 12, 128, 256
    x = _inputs(dev, B, S, H, 4, 64, W, 8, 8, 91)
    sm = 128 ** -0.5
    from aetherkv.decode import decode_workspace

    ws = decode_workspace(B, S, k, H, 128, W, dev)
    out = torch.empty((B, H, 128), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((B, k), dtype=torch.int64, device=dev)

    def step():
        csa_decode_step(x["q"], x["iq"], x["iw"], x["ix_codes"], x["ix_scale"], x["kv_codes"], x["kv_scale"], x["win"],
                        x["sink"], sm, k, kv_quant=x["kvq"], index_quant=x["ixq"], workspace=ws, out_idx=idx, out=out)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for r in range(3):
        x["iq"].copy_(normal((B, 4, 64), 300 + r, dtype=torch.float32, device=dev))
        x["q"].copy_(normal((B, 1, H, 128), 400 + r, device=dev))
        g.replay()
        torch.cuda.synchronize()
        got_o, got_i = out.clone(), idx.clone()
        step()
        torch.cuda.synchronize()
        assert torch.equal(got_i, idx) and torch.equal(got_o, out), f"replay {r}"
