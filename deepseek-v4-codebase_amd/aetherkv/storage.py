"""Quantised storage formats: paged-allocator pages and prefix-cache files holding TurboQuant codes
and scales instead of dequantised tensors.

What the reference does:
  * paging: _flush_live_page_if_ready / _flush_all_completed_pages (aether_2b/serving.py:857-905,
    1198-1273) dequantise each page's blocks to the model dtype (_compressed_to_bf16_for_paging,
    :378-398) before PagedKVAllocator.append_page (aether_kernels/paged_kv_allocator.py:121-136);
    the page shape is {"layer{i}.hca": (hca_blocks_per_page, D), "layer{i}.csa": (csa_blocks_per_page,
    D), "layer{i}.csa_index": (csa_blocks_per_page, IC)} in that dtype (allocator_page_shape,
    :403-410), and _materialize_paged_prefix (:486-493) concatenates the pages in front of the
    resident blocks;
  * prefix cache: ModelServingState.to_compressed_dict (:242-263) collects each layer's compressed
    tensors and scales on the CPU, and the prefix store torch.save()s that dict and reads it back with
    torch.load(weights_only=False) (aether_pipeline/serving.py:229-300).

Here a page row is one block's code bytes followed by its fp32 scale (little endian), so one
stream of a page is uint8 [blocks, row_bytes + 4]: the reference allocator is used unchanged with
dtype=torch.uint8 and the shapes from code_page_shape(), a page is 3.8x (4-bit) or 1.9x (8-bit)
smaller than its bf16 form, and pages go back into a CodeRing as codes, bit for bit, with no
decode/encode on either side.  Prefix files are safetensors (tensors + JSON metadata; loading
executes nothing from the file) with the same dict structure as to_compressed_dict.
"""
from __future__ import annotations

import json
from pathlib import Path
from typing import Dict, Mapping, Optional, Sequence, Tuple, Union

import torch

from .cache import CodeRing
from .turbo_quant import PolarQuant

FORMAT = "aetherkv.compressed_prefix.v1"
_LAYER_KEYS = ("compressed", "compressed_scale", "index_compressed", "index_compressed_scale")


def row_bytes(dim: int, bits: int) -> int:
    """Code bytes of one block of `dim` values (turbo_quant.py:150-166)."""
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    return dim if bits == 8 else dim // 2


def code_page_shape(page_shape: Mapping[str, Tuple[int, int]], bits: int) -> Dict[str, Tuple[int, int]]:
    """uint8 page shapes for the allocator from the engine's {name: (blocks, dim)} page shape."""
    return {name: (int(blocks), row_bytes(int(dim), bits) + 4) for name, (blocks, dim) in page_shape.items()}


def pack_rows(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """codes [m, row_bytes] (int8 or uint8) + scales [m] or [m, 1] fp32 -> uint8 [m, row_bytes + 4]."""
    if codes.dim() != 2 or codes.dtype not in (torch.int8, torch.uint8):
        raise RuntimeError(f"codes must be int8/uint8 [m, row_bytes], got {codes.dtype} {tuple(codes.shape)}")
    m = codes.size(0)
    if scale.numel() != m or scale.dtype != torch.float32:
        raise RuntimeError(f"scale must be fp32 with {m} values, got {scale.dtype} {tuple(scale.shape)}")
    sb = scale.reshape(m).contiguous().view(torch.uint8).view(m, 4)
    return torch.cat([codes.contiguous().view(torch.uint8), sb], dim=1)


def unpack_rows(page: torch.Tensor, bits: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """uint8 [m, row_bytes + 4] -> (codes [m, row_bytes] int8 (8-bit) or uint8 (4-bit), scales [m, 1] fp32)."""
    if page.dim() != 2 or page.dtype != torch.uint8 or page.size(1) < 5:
        raise RuntimeError(f"a code page is uint8 [m, row_bytes + 4], got {page.dtype} {tuple(page.shape)}")
    rb = page.size(1) - 4
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    codes = page[:, :rb].contiguous()
    if bits == 8:
        codes = codes.view(torch.int8)
    scale = page[:, rb:].contiguous().view(torch.float32).view(page.size(0), 1)
    return codes, scale


def flush_page(rings: Mapping[str, CodeRing], blocks_per_page: Mapping[str, int]) -> Dict[str, torch.Tensor]:
    """One page from the first blocks_per_page[name] blocks of each single-sequence ring, which are then
    dropped from the rings (the engine's page flush, serving.py:857-905).  Every ring is checked
    first: if any holds fewer blocks than its page needs, nothing changes and ValueError is raised."""
    for name, ring in rings.items():
        if ring.batch != 1:
            raise RuntimeError(f"pages hold one sequence; ring {name!r} has batch {ring.batch}")
        if name not in blocks_per_page:
            raise KeyError(f"no blocks_per_page entry for {name!r}")
        if ring.n < int(blocks_per_page[name]):
            raise ValueError(f"ring {name!r} holds {ring.n} blocks, a page needs {blocks_per_page[name]}")
    page = {}
    for name, ring in rings.items():
        m = int(blocks_per_page[name])
        page[name] = pack_rows(ring.data[0, :m], ring.scale[0, :m])
    for name, ring in rings.items():
        ring.drop_front(int(blocks_per_page[name]))
    return page


def materialize_pages(pages: Sequence[Mapping[str, torch.Tensor]], name: str, quant: PolarQuant, dim: int, *,
                      resident: Optional[CodeRing] = None, device=None, capacity: int = 0) -> CodeRing:
    """A ring holding stream `name` of the pages in order, followed by the resident ring's blocks (the
    paged prefix in front of the resident blocks, serving.py:486-493 and :786-798)."""
    rb = row_bytes(dim, quant.bits)
    parts = []
    for i, p in enumerate(pages):
        t = p[name]
        if t.dim() != 2 or t.size(1) != rb + 4:
            raise RuntimeError(f"page {i} stream {name!r} has shape {tuple(t.shape)}, expected [blocks, {rb + 4}]")
        parts.append(t)
    if device is None:
        device = resident.device if resident is not None else (parts[0].device if parts else None)
    n_paged = sum(t.size(0) for t in parts)
    n_res = resident.n if resident is not None else 0
    ring = CodeRing(quant, 1, dim, capacity=max(int(capacity), n_paged + n_res, 1), device=device)
    if parts:
        codes, scale = unpack_rows(torch.cat([t.to(device) for t in parts], dim=0), quant.bits)
        ring.append_codes(codes.unsqueeze(0), scale.unsqueeze(0))
    if resident is not None and resident.n:
        if resident.batch != 1 or resident.dim != dim or resident.quant.bits != quant.bits:
            raise RuntimeError("the resident ring must be a single-sequence ring of the same dim and bits")
        ring.append_codes(resident.data, resident.scale)
    return ring


def compressed_dict(layers: Sequence[Mapping[str, object]], reusable_tokens: int) -> Dict[str, object]:
    """to_compressed_dict (serving.py:242-263) from rings: layers are {"type": "hca", "kv": ring} or
    {"type": "csa", "kv": ring, "index": ring}; every tensor is moved to the CPU."""
    out = []
    for i, layer in enumerate(layers):
        kind = layer.get("type")
        if kind not in ("hca", "csa"):
            raise ValueError(f"layer {i}: type must be 'hca' or 'csa', got {kind!r}")
        kv: Optional[CodeRing] = layer.get("kv")
        entry = {"type": kind,
                 "compressed": None if kv is None else kv.data.cpu(),
                 "compressed_scale": None if kv is None else kv.scale.cpu()}
        if kind == "csa":
            ix: Optional[CodeRing] = layer.get("index")
            entry["index_compressed"] = None if ix is None else ix.data.cpu()
            entry["index_compressed_scale"] = None if ix is None else ix.scale.cpu()
        out.append(entry)
    return {"token_count": int(reusable_tokens), "layers": out}


def save_compressed_prefix(path: Union[str, Path], payload: Mapping[str, object], *, bits: int, seed: int = 42,
                           index_bits: Optional[int] = None) -> None:
    """Write a compressed-prefix dict (to_compressed_dict structure) as one safetensors file."""
    from safetensors.torch import save_file

    layers = payload["layers"]
    tensors: Dict[str, torch.Tensor] = {}
    types = []
    for i, layer in enumerate(layers):
        types.append(layer["type"])
        for key in _LAYER_KEYS:
            t = layer.get(key)
            if t is not None:
                tensors[f"layers.{i}.{key}"] = t.detach().to("cpu").contiguous()
    meta = {"format": FORMAT, "token_count": str(int(payload["token_count"])), "layer_types": json.dumps(types),
            "bits": str(int(bits)), "index_bits": str(int(index_bits if index_bits is not None else bits)),
            "seed": str(int(seed))}
    save_file(tensors, str(path), metadata=meta)


def load_compressed_prefix(path: Union[str, Path], device="cpu") -> Tuple[Dict[str, object], Dict[str, object]]:
    """Read a file written by save_compressed_prefix: (payload in to_compressed_dict structure,
    {"bits", "index_bits", "seed"}).  Raises ValueError for a file of another format."""
    from safetensors import safe_open

    with safe_open(str(path), framework="pt", device=str(device)) as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: not an {FORMAT} file (format {meta.get('format')!r})")
        types = json.loads(meta["layer_types"])
        names = set(f.keys())
        layers = []
        for i, kind in enumerate(types):
            entry: Dict[str, object] = {"type": kind}
            keys = _LAYER_KEYS if kind == "csa" else _LAYER_KEYS[:2]
            for key in keys:
                name = f"layers.{i}.{key}"
                entry[key] = f.get_tensor(name) if name in names else None
            layers.append(entry)
    info = {"bits": int(meta["bits"]), "index_bits": int(meta["index_bits"]), "seed": int(meta["seed"])}
    return {"token_count": int(meta["token_count"]), "layers": layers}, info
