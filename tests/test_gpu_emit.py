"""GPU tests of block emission (aekv_emit_block): the pooled, rotated, normalised vector against the
oracle, the codes against PolarQuant.encode of that vector, and the ring slot it lands in."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from aetherkv import PolarQuant
from aetherkv.cache import CodeRing, emit_block, rope_inv_freq
from conftest import bf16_bits

pytestmark = pytest.mark.gpu


def _inputs(dev, B, L, D, seed, bias=False, first_csa=False):
    g = torch.Generator(device=dev).manual_seed(seed)
    c = torch.randn(B, L, D, device=dev, generator=g).to(torch.bfloat16)
    z = (torch.randn(B, L, D, device=dev, generator=g) * 2).to(torch.bfloat16)
    b = (torch.randn(L, D, device=dev, generator=g) * 0.5).to(torch.bfloat16) if bias else None
    if first_csa:
        c[:, L // 2:] = 0
        z[:, L // 2:] = float("-inf")
    nw = (torch.rand(D, device=dev, generator=g) * 2).to(torch.bfloat16)
    return c, z, b, nw


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("case", ["hca", "csa_main", "csa_main_first", "csa_index"])
def test_emit_block_matches_oracle_and_encodes_exactly(dev, bits, case):
    B, m = 7, 128
    D = 64 if case == "csa_index" else 128
    L = m if case == "hca" else 2 * m
    c, z, bias, nw = _inputs(dev, B, L, D, 31 + bits, bias=case != "hca", first_csa=case == "csa_main_first")
    rope = 0 if case == "csa_index" else 64
    norm = None if case == "csa_index" else nw
    pos = torch.tensor([0, 127, 255, 4095, 65535, 131071, 262143], dtype=torch.int64)
    inv = rope_inv_freq(64, 10000.0)
    pq = PolarQuant(bits)
    codes, scale, vec = emit_block(pq, c, z, bias=bias, rope_dim=rope, positions=pos if rope else None,
                                   inv_freq=inv if rope else None, norm_weight=norm, return_vector=True)
    want = O.emit_block(bf16_bits(c), bf16_bits(z), None if bias is None else bf16_bits(bias), rope,
                        pos.numpy() if rope else None, inv.numpy() if rope else None,
                        None if norm is None else bf16_bits(norm), 1e-6)
    got = bf16_bits(vec).astype(np.int32)
    # device and host libm (exp, cos, sin) and the RMS sum order may differ by an fp32 ulp before a
    # bf16 rounding: at most one bf16 ulp, and nearly all bits equal
    assert np.all(np.abs(got - want.astype(np.int32)) <= 1)
    assert np.mean(got == want) > 0.99
    # the codes are exactly PolarQuant.encode of the emitted vector
    c2, s2 = pq.encode(vec)
    assert torch.equal(codes.view(B, -1), c2) and torch.equal(scale.view(B, 1), s2)


def test_append_emitted_writes_the_next_ring_slot(dev):
    B, D, L = 3, 128, 128
    pq = PolarQuant(4)
    ring = CodeRing(pq, B, D, capacity=2, device=dev)
    inv = rope_inv_freq(64, 10000.0)
    vecs = []
    for blk in range(5):  # grows the ring twice
        c, z, _, nw = _inputs(dev, B, L, D, 100 + blk)
        pos = torch.full((B,), 128 * blk + 127, dtype=torch.int64)
        ring.append_emitted(c, z, rope_dim=64, positions=pos, inv_freq=inv, norm_weight=nw)
        _, _, v = emit_block(pq, c, z, rope_dim=64, positions=pos, inv_freq=inv, norm_weight=nw, return_vector=True)
        vecs.append(v)
    assert ring.n == 5 and ring.capacity == 8
    c_all, s_all = pq.encode(torch.stack(vecs, dim=1))
    assert torch.equal(ring.data, c_all) and torch.equal(ring.scale, s_all)


def test_emit_block_argument_errors(dev):
    pq = PolarQuant(4)
    c = torch.zeros(2, 4, 96, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="head dim"):
        emit_block(pq, c, c)
    c = torch.zeros(2, 4, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="rope_dim"):
        emit_block(pq, c, c, rope_dim=64)
