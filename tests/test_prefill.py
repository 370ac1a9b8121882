"""CPU tests of the chunked-prefill bookkeeping (aetherkv.prefill.prefill_sources): which compressed
blocks and sliding-window entries each target sees, as modeling.py:316-320 / :521-534 define them
(g = min(nb, t // M); window [max(0, t - W + 1), t]), and the host-side argument checks."""
from __future__ import annotations

import pytest
import torch

from aetherkv.prefill import prefill_sources, quant_prefill_attention


def _l(t: torch.Tensor):
    return t.tolist()


def test_first_chunk_small_case():
    # positions 0..9, M = 4, W = 3, 2 blocks emitted so far, window buffer = positions 0..9
    vis, ws, wl = prefill_sources(10, 0, 2, compression=4, sliding_window=3, window_base=0, window_len=10)
    assert _l(vis) == [0, 0, 0, 0, 1, 1, 1, 1, 2, 2]  # t // 4, capped at 2 blocks
    assert _l(ws) == [0, 0, 0, 1, 2, 3, 4, 5, 6, 7]   # max(0, t - 2)
    assert _l(wl) == [1, 2, 3, 3, 3, 3, 3, 3, 3, 3]
    assert vis.dtype == ws.dtype == wl.dtype == torch.int32


def test_later_chunk_with_window_history():
    # chunk of positions 300..303 with M = 128, W = 128: the first target's window starts at 173, so
    # the buffer holds the W - 1 entries before the chunk plus its T entries: positions 173..303
    vis, ws, wl = prefill_sources(4, 300, 100, compression=128, sliding_window=128, window_base=173,
                                  window_len=131)
    assert _l(vis) == [2, 2, 2, 2]
    assert _l(ws) == [0, 1, 2, 3]
    assert _l(wl) == [128, 128, 128, 128]
    # the same chunk against a buffer that starts 10 positions earlier
    _, ws, _ = prefill_sources(4, 300, 100, compression=128, sliding_window=128, window_base=163, window_len=141)
    assert _l(ws) == [10, 11, 12, 13]


def test_block_boundary_and_block_cap():
    # a target at position 127 sees no HCA block; 128 sees one; a cap of 0 emitted blocks wins
    vis, _, _ = prefill_sources(3, 127, 5, compression=128, sliding_window=128, window_base=0, window_len=130)
    assert _l(vis) == [0, 1, 1]
    vis, _, _ = prefill_sources(3, 127, 0, compression=128, sliding_window=128, window_base=0, window_len=130)
    assert _l(vis) == [0, 0, 0]


def test_window_buffer_must_cover_every_slice():
    with pytest.raises(ValueError):  # position 5 needs entries from 3, the buffer starts at 4
        prefill_sources(2, 5, 1, compression=4, sliding_window=3, window_base=4, window_len=10)
    with pytest.raises(ValueError):  # the buffer ends before the last target
        prefill_sources(4, 0, 1, compression=4, sliding_window=3, window_base=0, window_len=3)
    with pytest.raises(ValueError):
        prefill_sources(1, -1, 1, compression=4, sliding_window=3, window_base=0, window_len=3)
    vis, ws, wl = prefill_sources(0, 7, 1, compression=4, sliding_window=3, window_base=0, window_len=0)
    assert vis.numel() == ws.numel() == wl.numel() == 0


def test_attention_rejects_host_tensors():
    from aetherkv import PolarQuant

    q = torch.zeros(1, 2, 4, 128, dtype=torch.bfloat16)
    codes = torch.zeros(1, 3, 64, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="HIP device"):
        quant_prefill_attention(q, codes, torch.ones(1, 3), None, None, torch.zeros(4), 0.1, quant=PolarQuant(4))
