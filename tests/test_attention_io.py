"""CPU tests for the query/output-side work around attention: the oracle's RoPE + RMSNorm
(oracle.rope_rmsnorm) pinned against the reference's torch op sequence (apply_rope
modeling.py:122-155 with _rotate_half, F.rms_norm as RMSNorm :32-41), the host-side position
handling, and the grouped output projection against a block-diagonal formulation."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from aetherkv.attention_io import _row_positions, grouped_output_projection
from conftest import bf16_bits


def _torch_rope_norm(x, pos, rope, inv_freq, w, eps, sign):
    """The reference's op sequence on the CPU (bf16 tensors; cos/sin from fp32 angles)."""
    rows, H, D = x.shape
    if rope:
        pp, rp = x[..., :-rope], x[..., -rope:]
        ang = (sign * pos).float().unsqueeze(-1) * inv_freq
        cos = torch.repeat_interleave(ang.cos(), 2, dim=-1).to(x.dtype).view(rows, 1, rope)
        sin = torch.repeat_interleave(ang.sin(), 2, dim=-1).to(x.dtype).view(rows, 1, rope)
        x1, x2 = rp[..., ::2], rp[..., 1::2]
        rot = torch.stack((-x2, x1), dim=-1).flatten(-2)
        x = torch.cat([pp, rp * cos + rot * sin], dim=-1)
    if w is not None:
        x = F.rms_norm(x, (D,), w, eps)
    return x


@pytest.mark.parametrize("D,rope,norm,sign", [(128, 64, True, 1), (128, 64, False, -1), (128, 0, True, 1),
                                              (128, 128, True, 1), (256, 64, True, 1), (256, 32, False, -1)])
def test_oracle_rope_rmsnorm_matches_torch_op_sequence(D, rope, norm, sign):
    g = torch.Generator().manual_seed(D + rope + sign)
    rows, H = 6, 5
    x = (torch.randn(rows, H, D, generator=g) * 3).to(torch.bfloat16)
    pos = torch.tensor([0, 1, 127, 4096, 65535, 262143])
    inv = 1.0 / (10000.0 ** (torch.arange(0, max(rope, 2), 2, dtype=torch.float32) / max(rope, 2)))
    w = (torch.rand(D, generator=g) * 2).to(torch.bfloat16) if norm else None
    want = bf16_bits(_torch_rope_norm(x, pos, rope, inv, w, 1e-6, sign))
    got = O.rope_rmsnorm(bf16_bits(x), pos.numpy(), inv.numpy() if rope else None, rope,
                         None if w is None else bf16_bits(w), 1e-6, sign)
    d = np.abs(got.astype(np.int32) - want.astype(np.int32))
    # torch's CPU reduction order for the mean can move r by an fp32 ulp: at most one bf16 ulp
    assert d.max() <= 1 and np.mean(d == 0) > 0.995


def test_oracle_rope_is_a_rotation():
    # rope then inverse rope returns the input up to the bf16 roundings; angle 0 is the identity
    x = torch.randn(2, 3, 128).to(torch.bfloat16)
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    same = O.rope_rmsnorm(bf16_bits(x), np.zeros(2, np.int64), inv.numpy(), 64)
    np.testing.assert_array_equal(same, bf16_bits(x))
    pos = np.array([300, 9000], np.int64)
    fwd = O.rope_rmsnorm(bf16_bits(x), pos, inv.numpy(), 64)
    back = O.rope_rmsnorm(fwd, pos, inv.numpy(), 64, sign=-1)
    xb = O.bf16_to_f32(bf16_bits(x))
    np.testing.assert_allclose(O.bf16_to_f32(back), xb, atol=0.06 * np.abs(xb).max())
    np.testing.assert_array_equal(O.bf16_to_f32(back)[..., :64], xb[..., :64])  # pass-through part untouched


def test_row_positions():
    dev = torch.device("cpu")
    assert _row_positions(7, (2, 3), dev).tolist() == [7] * 6
    assert _row_positions(torch.tensor([4, 5, 6]), (2, 3), dev).tolist() == [4, 5, 6, 4, 5, 6]
    assert _row_positions(torch.tensor([[1, 2, 3], [4, 5, 6]]), (2, 3), dev).tolist() == [1, 2, 3, 4, 5, 6]
    assert _row_positions(torch.tensor(9), (4,), dev).tolist() == [9] * 4
    with pytest.raises(RuntimeError):
        _row_positions(torch.tensor([1, 2]), (2, 3), dev)


def test_grouped_output_projection_equals_block_diagonal_matrix():
    torch.manual_seed(3)
    B, H, D, G, go, hidden = 5, 8, 16, 4, 12, 20
    x = torch.randn(B, H, D, dtype=torch.float64)
    gw = [torch.randn(go, H // G * D, dtype=torch.float64) for _ in range(G)]
    ow = torch.randn(hidden, G * go, dtype=torch.float64)
    bd = torch.block_diag(*gw)  # [G*go, H*D]: group g reads heads g*H/G .. (g+1)*H/G - 1
    want = x.reshape(B, H * D) @ bd.T @ ow.T
    got = grouped_output_projection(x, gw, ow)
    torch.testing.assert_close(got, want)
    with pytest.raises(RuntimeError):
        grouped_output_projection(x, gw[:3], ow)
