"""CPU tests of aetherkv.cache: the engine's state types and quant helpers (aether_2b/serving.py:32-37,
66-214, 327-398) and CodeRing's placement and growth logic (with an oracle-backed quantiser on the
CPU; the GPU path is in test_gpu_cache.py)."""
from __future__ import annotations

from dataclasses import fields

import numpy as np
import pytest
import torch

import oracle as O
from aetherkv.cache import (CodeRing, CSAServingState, DequantMemo, HCAServingState, append_seq,
                            block_rope_position, compressed_to_bf16_for_paging, quant_append, read_compressed,
                            rope_inv_freq)
from conftest import bf16_bits

HCA_FIELDS = ["token_count", "loaded_prefix_tokens", "compressed", "compressed_scale", "window", "buffer_c",
              "buffer_z"]  # serving.py:66-74
CSA_FIELDS = ["token_count", "loaded_prefix_tokens", "compressed", "compressed_scale", "index_compressed",
              "index_compressed_scale", "window", "curr_a_c", "curr_a_z", "curr_b_c", "curr_b_z", "curr_index_a_c",
              "curr_index_a_z", "curr_index_b_c", "curr_index_b_z", "prev_b_c", "prev_b_z", "prev_index_b_c",
              "prev_index_b_z"]  # serving.py:112-131


def test_state_fields_match_the_engine():
    assert [f.name for f in fields(HCAServingState)] == HCA_FIELDS
    assert [f.name for f in fields(CSAServingState)] == CSA_FIELDS
    assert HCAServingState().token_count == 0 and CSAServingState().compressed is None


@pytest.mark.parametrize("cls,kind", [(HCAServingState, "hca"), (CSAServingState, "csa")])
def test_state_to_dict_from_dict_and_clone(cls, kind):
    names = [f.name for f in fields(cls) if f.name not in ("token_count", "loaded_prefix_tokens")]
    st = cls(token_count=300, loaded_prefix_tokens=128)
    for i, n in enumerate(names[::2]):  # every other tensor field set, the rest None
        setattr(st, n, torch.full((2, 3), float(i)))
    d = st.to_dict()
    assert d["type"] == kind and d["token_count"] == 300 and d["loaded_prefix_tokens"] == 128
    assert set(d) == {"type", "token_count", "loaded_prefix_tokens", *names}
    back = cls.from_dict(d, torch.device("cpu"))
    for n in names:
        a, b = getattr(st, n), getattr(back, n)
        assert (a is None and b is None) or torch.equal(a, b)
    # loaded_prefix_tokens defaults to 0; token_count is required
    d2 = dict(d)
    del d2["loaded_prefix_tokens"]
    assert cls.from_dict(d2, torch.device("cpu")).loaded_prefix_tokens == 0
    del d2["token_count"]
    with pytest.raises(KeyError):
        cls.from_dict(d2, torch.device("cpu"))
    # clone is deep
    c = st.clone()
    getattr(c, names[0]).fill_(-5.0)
    assert float(getattr(st, names[0])[0, 0]) == 0.0 and c.token_count == 300


def test_append_seq_and_passthrough_helpers():
    a = append_seq(None, torch.ones(2, 4))
    assert a.shape == (2, 1, 4)
    b = append_seq(a, torch.zeros(2, 3, 4))
    assert b.shape == (2, 4, 4) and float(b[:, 0].sum()) == 8.0 and float(b[:, 1:].sum()) == 0.0
    x = torch.randn(2, 5, 8)
    d, s = quant_append(None, None, None, x)
    assert s is None and torch.equal(d, x)
    assert read_compressed(None, x, None, torch.bfloat16) is x
    assert read_compressed(None, None, None, torch.bfloat16) is None
    assert compressed_to_bf16_for_paging(None, x, None, 1, 3, torch.bfloat16).shape == (2, 2, 8)
    assert compressed_to_bf16_for_paging(None, x, None, 1, 6, torch.bfloat16) is None  # fewer blocks than end


def test_dequant_memo_is_bounded_and_cleared_when_full():
    m = DequantMemo(limit=3)
    for i in range(3):
        m.put(("k", i), torch.zeros(1))
    assert len(m) == 3
    m.put(("k", 3), torch.ones(1))  # full: everything is dropped, then the new entry kept
    assert len(m) == 1 and m.get(("k", 0)) is None and m.get(("k", 3)) is not None
    t = torch.zeros(2, 3)
    s = torch.zeros(2, 1)
    assert DequantMemo.key(t, s, torch.bfloat16) == (t.data_ptr(), (2, 3), s.data_ptr(), (2, 1), "torch.bfloat16")


class OracleQuant:
    """CPU stand-in for PolarQuant with the oracle's encode (test infrastructure only)."""

    def __init__(self, bits: int):
        self.bits = bits

    def encode(self, x: torch.Tensor):
        d = x.shape[-1]
        c, s = O.encode(bf16_bits(x.to(torch.bfloat16)).reshape(-1, d), "bf16", self.bits, O.diag(42, d))
        lead = tuple(x.shape[:-1])
        return torch.from_numpy(c).reshape(lead + (c.shape[-1],)), torch.from_numpy(s).reshape(lead + (1,))


@pytest.mark.parametrize("bits", [4, 8])
def test_code_ring_appends_in_place_and_grows(bits):
    B, D = 3, 64
    q = OracleQuant(bits)
    ring = CodeRing(q, B, D, capacity=4, device=torch.device("cpu"))
    g = torch.Generator().manual_seed(bits)
    blocks = []
    storage0 = ring.storage[0].data_ptr()
    for m in [1, 1, 2, 3, 1, 5, 0, 2]:
        new = torch.randn(B, m, D, generator=g).to(torch.bfloat16)
        ring.append(new if m != 1 else new[:, 0])  # [B, D] appends one block
        blocks.append(new)
    allx = torch.cat(blocks, dim=1)
    n = allx.size(1)
    assert ring.n == n and ring.capacity >= n
    assert ring.capacity == 16  # 4 -> 8 -> 16 (doubling)
    assert ring.storage[0].data_ptr() != storage0
    want_c, want_s = q.encode(allx)
    assert torch.equal(ring.data, want_c) and torch.equal(ring.scale, want_s)
    assert torch.equal(ring.visible(), torch.full((B,), n, dtype=torch.int32))
    assert torch.equal(ring.all_indices(), torch.arange(n).expand(B, n))
    assert ring.all_indices().is_contiguous()
    # slots past n are zero (finite values for anything that reads the whole storage)
    assert int(ring.storage[0][:, n:].abs().sum()) == 0 and float(ring.storage[1][:, n:].abs().sum()) == 0.0
    again = CodeRing.from_tensors(q, ring.data, ring.scale, capacity=40)
    assert again.n == n and again.capacity == 40 and torch.equal(again.data, ring.data)


def test_code_ring_rejects_bad_shapes():
    ring = CodeRing(OracleQuant(8), 2, 16, capacity=2, device=torch.device("cpu"))
    with pytest.raises(RuntimeError):
        ring.append(torch.zeros(3, 16))
    with pytest.raises(RuntimeError):
        ring.append(torch.zeros(2, 1, 8))
    with pytest.raises(ValueError):
        CodeRing(OracleQuant(8), 0, 16, device=torch.device("cpu"))


def test_block_rope_position_conventions():
    m = 128
    blocks = torch.arange(6)
    # the engine emits block i when token_count reaches (i + 1) m and passes token_count - 1
    # (serving.py:534, :640); HCA rotates at it (:498), the step-by-step CSA emission at it - (m - 1) (:564)
    emitted_at = (blocks + 1) * m - 1
    assert torch.equal(block_rope_position(blocks, m), emitted_at)
    assert torch.equal(block_rope_position(blocks, m, "start"), emitted_at - (m - 1))
    # the model's and the batched prefill's CSA blocks: arange(n) * m + (m - 1) (modeling.py:480)
    assert torch.equal(block_rope_position(blocks, m), torch.arange(6) * m + (m - 1))
    assert block_rope_position(3, 4) == 15 and block_rope_position(3, 4, "start") == 12
    with pytest.raises(ValueError):
        block_rope_position(1, m, "middle")


@pytest.mark.parametrize("block", [0, 5, 300])
def test_end_position_puts_a_new_block_at_distance_one(block):
    """RoPE scores depend on the position difference only: the query at (i + 1) m, the first that
    sees block i, scores that block's key as a key at distance 1 under "end" and m under "start"
    (the distance the reference's modeling.py:476-478 comment names)."""
    m, D, rd = 128, 128, 64
    rng = np.random.default_rng(11 + block)
    q = O.f32_to_bf16(rng.standard_normal((1, 1, D)).astype(np.float32))
    k = O.f32_to_bf16(rng.standard_normal((1, 1, D)).astype(np.float32))
    inv = rope_inv_freq(rd, 10000.0).numpy()
    f32 = lambda u: O.bf16_to_f32(u).astype(np.float64).ravel()
    tol = 0.02 * np.linalg.norm(f32(q)) * np.linalg.norm(f32(k))
    t = (block + 1) * m
    qt = f32(O.rope_rmsnorm(q, np.array([t]), inv, rd))
    for conv, dist, other in (("end", 1, m), ("start", m, 1)):
        kp = f32(O.rope_rmsnorm(k, np.array([block_rope_position(block, m, conv)]), inv, rd))
        score = qt @ kp
        at = lambda d: f32(O.rope_rmsnorm(q, np.array([d]), inv, rd)) @ f32(k)
        assert abs(score - at(dist)) <= tol
        assert abs(score - at(other)) > tol  # and the two conventions are told apart
