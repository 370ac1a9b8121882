"""GPU tests of aekv_rope_rmsnorm and the query/output-side helpers (aetherkv.attention_io) against
the oracle, which is pinned to the reference's torch op sequence on the CPU."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from aetherkv.attention_io import post_attention, query_prep, rope_rmsnorm, window_entry
from aetherkv.cache import rope_inv_freq
from conftest import bf16_bits

pytestmark = pytest.mark.gpu


def _close_bits(got: torch.Tensor, want: np.ndarray):
    """Nearly all bits equal; elsewhere within one bf16 ulp of the vector's largest element.

    Device and host cos/sin (and the RMS sum order) can differ by an fp32 ulp; where that straddles
    a bf16 tie, bf16(cos) or bf16(sin) differs by one bf16 ulp, and the rotated pair moves by up to
    |partner| * 2^-8 — many ulps of an element that nearly cancels, never more than that bound."""
    g = bf16_bits(got)
    d = g.astype(np.int32) != want.astype(np.int32)
    assert np.mean(~d) > 0.99
    gv = O.bf16_to_f32(g).reshape(-1, want.shape[-1])
    wv = O.bf16_to_f32(want).reshape(-1, want.shape[-1])
    bound = 2.0 ** -7 * np.abs(wv).max(axis=1, keepdims=True)
    assert np.all(np.abs(gv - wv) <= bound)


@pytest.mark.parametrize("D,rope,norm,inverse", [(128, 64, True, False), (128, 64, False, True),
                                                 (128, 0, True, False), (128, 128, True, False),
                                                 (256, 64, True, False), (256, 96, False, True)])
def test_rope_rmsnorm_matches_oracle(dev, D, rope, norm, inverse):
    g = torch.Generator(device=dev).manual_seed(D + rope)
    rows, H = 37, 12
    x = (torch.randn(rows, H, D, device=dev, generator=g) * 3).to(torch.bfloat16)
    pos = torch.randint(0, 262144, (rows,), device=dev, generator=g)
    pos[:3] = torch.tensor([0, 1, 262143], device=dev)
    inv = rope_inv_freq(max(rope, 2), 10000.0).to(dev)
    w = (torch.rand(D, device=dev, generator=g) * 2).to(torch.bfloat16) if norm else None
    got = rope_rmsnorm(x, pos, rope_dim=rope, inv_freq=inv if rope else None, norm_weight=w, inverse=inverse)
    want = O.rope_rmsnorm(bf16_bits(x), pos.cpu().numpy(), inv.cpu().numpy() if rope else None, rope,
                          None if w is None else bf16_bits(w), 1e-6, -1 if inverse else 1)
    _close_bits(got, want)
    # in place (out aliases x) gives the same bits
    x2 = x.clone()
    rope_rmsnorm(x2, pos, rope_dim=rope, inv_freq=inv if rope else None, norm_weight=w, inverse=inverse, out=x2)
    assert torch.equal(x2, got)


def test_query_window_and_post_attention_compose(dev):
    B, T, H, D, hidden, G, go = 4, 3, 16, 128, 1536, 4, 384
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn(B, T, H, D, device=dev, generator=g).to(torch.bfloat16)
    kv = torch.randn(B, T, D, device=dev, generator=g).to(torch.bfloat16)
    qw = (torch.rand(D, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(D, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    inv = rope_inv_freq(64, 10000.0).to(dev)
    tpos = torch.tensor([1000, 1001, 1002])
    qp = query_prep(q, tpos, inv, rope_dim=64, q_norm_weight=qw)
    rows_pos = tpos.repeat(B).numpy()
    want = O.rope_rmsnorm(bf16_bits(q).reshape(B * T, H, D), rows_pos, inv.cpu().numpy(), 64, bf16_bits(qw))
    _close_bits(qp.reshape(B * T, H, D), want)
    we = window_entry(kv, tpos, inv, rope_dim=64, kv_norm_weight=kw)
    assert we.shape == (B, T, D)
    want = O.rope_rmsnorm(bf16_bits(kv).reshape(B * T, 1, D), rows_pos, inv.cpu().numpy(), 64, bf16_bits(kw))
    _close_bits(we.reshape(B * T, 1, D), want)
    # post attention: inverse rope then the grouped projection (library GEMMs on the rotated output)
    gw = [(torch.randn(go, H // G * D, device=dev, generator=g) * 0.02).to(torch.bfloat16) for _ in range(G)]
    ow = (torch.randn(hidden, G * go, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    y = post_attention(qp, tpos, inv, rope_dim=64, group_weights=gw, out_proj_weight=ow)
    assert y.shape == (B, T, hidden) and y.dtype == torch.bfloat16
    rot = O.rope_rmsnorm(bf16_bits(qp).reshape(B * T, H, D), rows_pos, inv.cpu().numpy(), 64, None, sign=-1)
    rot_t = torch.from_numpy(O.bf16_to_f32(rot)).reshape(B, T, H, D)
    chunks = rot_t.chunk(G, dim=-2)
    ref = torch.cat([c.flatten(-2) @ w.float().cpu().T for c, w in zip(chunks, gw)], dim=-1) @ ow.float().cpu().T
    torch.testing.assert_close(y.float().cpu(), ref, rtol=2e-2, atol=2e-2)
