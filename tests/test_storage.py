"""CPU tests of the quantised storage formats (aetherkv.storage): the code-page row layout, page
flush / materialisation through CodeRing (with an oracle-backed quantiser), and the safetensors
prefix file, against the reference engine's page and prefix conventions
(aether_2b/serving.py:242-263, 403-410, 486-493, 857-905)."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from aetherkv.cache import CodeRing
from aetherkv.storage import (code_page_shape, compressed_dict, flush_page, load_compressed_prefix,
                              materialize_pages, pack_rows, row_bytes, save_compressed_prefix, unpack_rows)
from test_cache import OracleQuant


def test_page_shapes_follow_the_engine_layout():
    # allocator_page_shape (serving.py:403-410) with 1 HCA block and 32 CSA blocks per 128-token page
    shape = {"layer0.hca": (1, 128), "layer1.csa": (32, 128), "layer1.csa_index": (32, 64)}
    assert code_page_shape(shape, 4) == {"layer0.hca": (1, 68), "layer1.csa": (32, 68), "layer1.csa_index": (32, 36)}
    assert code_page_shape(shape, 8) == {"layer0.hca": (1, 132), "layer1.csa": (32, 132), "layer1.csa_index": (32, 68)}
    bf16 = sum(b * d * 2 for b, d in shape.values())
    q4 = sum(b * w for b, w in code_page_shape(shape, 4).values())
    assert bf16 == 12544 and q4 == 3396  # 3.7x smaller per layer pair
    assert row_bytes(64, 4) == 32 and row_bytes(64, 8) == 64
    with pytest.raises(ValueError):
        row_bytes(64, 6)


def test_row_layout_is_codes_then_little_endian_scale():
    codes = torch.tensor([[1, 2, 3, 250], [0, 255, 7, 8]], dtype=torch.uint8)
    scale = torch.tensor([1.5, -0.25], dtype=torch.float32)
    page = pack_rows(codes, scale)
    assert page.dtype == torch.uint8 and page.shape == (2, 8)
    assert page[0, :4].tolist() == [1, 2, 3, 250]
    assert bytes(page[0, 4:].tolist()) == struct.pack("<f", 1.5)
    assert bytes(page[1, 4:].tolist()) == struct.pack("<f", -0.25)
    c, s = unpack_rows(page, 4)
    assert c.dtype == torch.uint8 and torch.equal(c, codes) and torch.equal(s.view(-1), scale)
    c8, _ = unpack_rows(pack_rows(codes.view(torch.int8), scale), 8)
    assert c8.dtype == torch.int8 and torch.equal(c8.view(torch.uint8), codes)
    with pytest.raises(RuntimeError):
        pack_rows(codes, scale[:1])
    with pytest.raises(RuntimeError):
        unpack_rows(page.view(torch.int8), 4)


@pytest.mark.parametrize("bits", [4, 8])
def test_flush_then_materialize_round_trips_the_codes(bits):
    D, IC = 64, 32
    q = OracleQuant(bits)
    kv = CodeRing(q, 1, D, capacity=4, device=torch.device("cpu"))
    ix = CodeRing(q, 1, IC, capacity=4, device=torch.device("cpu"))
    g = torch.Generator().manual_seed(bits)
    kv.append(torch.randn(1, 11, D, generator=g).to(torch.bfloat16))
    ix.append(torch.randn(1, 11, IC, generator=g).to(torch.bfloat16))
    all_kv = (kv.data.clone(), kv.scale.clone())
    all_ix = (ix.data.clone(), ix.scale.clone())
    pages = [flush_page({"layer1.csa": kv, "layer1.csa_index": ix}, {"layer1.csa": 4, "layer1.csa_index": 4})
             for _ in range(2)]
    assert kv.n == 3 and ix.n == 3
    assert torch.equal(kv.data, all_kv[0][:, 8:]) and torch.equal(ix.scale, all_ix[1][:, 8:])
    assert int(kv.storage[0][:, 3:].abs().sum()) == 0  # freed slots zeroed
    assert pages[0]["layer1.csa"].shape == (4, row_bytes(D, bits) + 4)
    # not enough blocks for a third page: nothing changes
    with pytest.raises(ValueError):
        flush_page({"layer1.csa": kv, "layer1.csa_index": ix}, {"layer1.csa": 4, "layer1.csa_index": 4})
    assert kv.n == 3 and ix.n == 3
    back = materialize_pages(pages, "layer1.csa", q, D, resident=kv)
    assert back.n == 11
    assert torch.equal(back.data, all_kv[0]) and torch.equal(back.scale, all_kv[1])
    back_ix = materialize_pages(pages, "layer1.csa_index", q, IC, resident=ix)
    assert torch.equal(back_ix.data, all_ix[0]) and torch.equal(back_ix.scale, all_ix[1])
    only_pages = materialize_pages(pages, "layer1.csa", q, D, device=torch.device("cpu"))
    assert only_pages.n == 8 and torch.equal(only_pages.data, all_kv[0][:, :8])


def test_flush_rejects_batched_rings():
    ring = CodeRing(OracleQuant(8), 2, 16, capacity=4, device=torch.device("cpu"))
    ring.append(torch.zeros(2, 4, 16))
    with pytest.raises(RuntimeError):
        flush_page({"x": ring}, {"x": 2})


def test_prefix_file_round_trip(tmp_path):
    q4, q8 = OracleQuant(4), OracleQuant(8)
    g = torch.Generator().manual_seed(9)
    hca = CodeRing(q4, 1, 64, device=torch.device("cpu"))
    hca.append(torch.randn(1, 3, 64, generator=g))
    kv = CodeRing(q4, 1, 64, device=torch.device("cpu"))
    kv.append(torch.randn(1, 5, 64, generator=g))
    ix = CodeRing(q8, 1, 32, device=torch.device("cpu"))
    ix.append(torch.randn(1, 5, 32, generator=g))
    payload = compressed_dict([{"type": "hca", "kv": hca}, {"type": "csa", "kv": kv, "index": ix},
                               {"type": "hca", "kv": None}], reusable_tokens=384)
    assert payload["token_count"] == 384 and payload["layers"][1]["index_compressed"].dtype == torch.int8
    path = tmp_path / "p.safetensors"
    save_compressed_prefix(path, payload, bits=4, index_bits=8, seed=42)
    back, info = load_compressed_prefix(path)
    assert info == {"bits": 4, "index_bits": 8, "seed": 42}
    assert back["token_count"] == 384 and [l["type"] for l in back["layers"]] == ["hca", "csa", "hca"]
    for a, b in zip(payload["layers"], back["layers"]):
        assert set(a) == set(b)
        for k in a:
            if k == "type":
                continue
            assert (a[k] is None and b[k] is None) or (a[k].dtype == b[k].dtype and torch.equal(a[k], b[k]))
    # a safetensors file of another format is refused
    from safetensors.torch import save_file
    other = tmp_path / "o.safetensors"
    save_file({"x": torch.zeros(2)}, str(other), metadata={"format": "something-else"})
    with pytest.raises(ValueError):
        load_compressed_prefix(other)
    with pytest.raises(ValueError):
        compressed_dict([{"type": "mla"}], 0)
