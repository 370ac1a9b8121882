"""GPU parity of the CSA indexer + top-k (fp32 drop-in and quantised keys) against the oracle.

Bar: the selected set equals the oracle's exact-math top-k, except for indices whose oracle score
is within the fp32 rounding bound of the k-th score (see topk_check.py); output sorted by score,
padded with -1 beyond the visible count; exact ties resolve to the lower index.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
from aetherkv import PolarQuant, csa_indexer_topk
from aetherkv.decode import csa_indexer_topk_quant
from aetherkv.synthetic import normal, normal_with_outliers
from topk_check import assert_topk_matches, score_error_bound

pytestmark = pytest.mark.gpu


def w_act(w: np.ndarray, mode: str) -> np.ndarray:
    w = w.astype(np.float64)
    if mode == "softplus":
        return np.where(w > 20, w, np.log1p(np.exp(np.minimum(w, 20))))
    return np.maximum(w, 0) if mode == "relu_w" else w


@pytest.mark.parametrize("mode", ["softplus", "raw", "relu_w"])
@pytest.mark.parametrize("S,k", [(1, 1), (7, 7), (300, 16), (5000, 256), (9000, 2048), (4096, 256)])
def test_fp32_indexer_matches_oracle(dev, mode, S, k):
    B, IH, IC = 3, 4, 64
    g = torch.Generator().manual_seed(S * 3 + k)
    q = torch.randn(B, IH, IC, generator=g)
    kv = torch.randn(B, S, IC, generator=g)
    w = torch.randn(B, IH, generator=g) * 2
    idx = csa_indexer_topk(q.to(dev), kv.to(dev), w.to(dev), k, mode=mode).cpu().numpy()
    assert idx.shape == (B, k) and idx.dtype == np.int64
    scores = O.index_scores(q.numpy(), w.numpy(), kv.numpy(), mode=mode)
    tol = score_error_bound(q.numpy(), w_act(w.numpy(), mode), kv.numpy())
    assert_topk_matches(idx, scores, k, tol)


def test_fp32_indexer_reference_contract(dev):
    # k must be in [1, S] (csa_indexer_cuda.cu:95); output int64 [B, k]
    q = torch.randn(1, 2, 8, device=dev)
    kv = torch.randn(1, 5, 8, device=dev)
    w = torch.randn(1, 2, device=dev)
    with pytest.raises(RuntimeError, match=r"k must be in \[1, S\]"):
        csa_indexer_topk(q, kv, w, 6)
    assert csa_indexer_topk(q, kv, w, 5).shape == (1, 5)


def test_exact_ties_pick_lowest_indices(dev):
    B, S, IH, IC = 2, 9000, 2, 16
    q = torch.randn(B, IH, IC)
    kv = torch.randn(1, 1, IC).expand(B, S, IC).contiguous()   # every key identical -> all scores tie
    w = torch.ones(B, IH)
    idx = csa_indexer_topk(q.to(dev), kv.to(dev), w.to(dev), 300).cpu().numpy()
    np.testing.assert_array_equal(idx, np.tile(np.arange(300), (B, 1)))


def _quant_case(dev, B, S, IH, IC, bits, seed, outliers=False, mode="softplus", k=256, valid=None):
    pq = PolarQuant(bits)
    keys = (normal_with_outliers((B, S, IC), seed, dtype=torch.bfloat16, trailing_dims=1) if outliers
            else normal((B, S, IC), seed, dtype=torch.bfloat16)).to(dev)
    codes, scale = pq.encode(keys)
    q = normal((B, IH, IC), seed + 100, dtype=torch.float32).to(dev)
    w = normal((B, IH), seed + 200, dtype=torch.float32).to(dev)
    vt = None if valid is None else torch.tensor(valid, dtype=torch.int32, device=dev)
    idx, sc = csa_indexer_topk_quant(q, w, codes, scale, k, quant=pq, valid=vt, mode=mode, return_scores=True)
    # oracle: keys dequantised in fp32 (turbo_quant.py decode), exact-math scores
    dg = O.diag(42, IC)
    keys_f32 = O.decode(codes.cpu().numpy(), scale.cpu().numpy(), bits, dg, "f32")
    qn, wn = q.cpu().numpy(), w.cpu().numpy()
    scores = O.index_scores(qn, wn, keys_f32, valid=None if valid is None else np.array(valid, np.int32), mode=mode)
    tol = score_error_bound(qn, w_act(wn, mode), keys_f32, extra_rel=16 * math.log2(IC) * 2.0 ** -24)
    subs = assert_topk_matches(idx.cpu().numpy(), scores, k, tol, None if valid is None else np.array(valid))
    # returned scores agree with the oracle's within the bound
    ii = idx.cpu().numpy()
    ok = ii >= 0
    bi = np.nonzero(ok)
    ref = scores[bi[0], ii[ok]]
    assert np.all(np.abs(sc.cpu().numpy()[ok] - ref) <= 2 * tol[bi[0], ii[ok]] + 1e-30)
    return subs


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("mode", ["softplus", "raw", "relu_w"])
def test_quant_indexer_matches_oracle(dev, bits, mode):
    _quant_case(dev, 3, 6000, 4, 64, bits, 10 + bits, mode=mode)


def test_quant_indexer_ragged_valid_and_padding(dev):
    _quant_case(dev, 4, 5000, 4, 64, 4, 21, valid=[5000, 2500, 0, 3], k=16)


def test_quant_indexer_small_dims(dev):
    # tiny-model shapes of the reference tests (indexer_head_dim=8, 2 heads)
    _quant_case(dev, 2, 37, 2, 8, 8, 31, k=4)
    _quant_case(dev, 2, 37, 2, 8, 4, 32, k=37)


def test_config3_indexer_8bit(dev):
    # benchmark configuration cfg3: B=8, 16384 blocks, 4 index heads x 64, 8-bit keys, softplus weights, top-256
    _quant_case(dev, 8, 16384, 4, 64, 8, 2)


def test_config5_indexer_4bit_rows(dev):
    # benchmark configuration cfg5 at full S (65536 blocks, 4-bit, outliers) on 2 of the 64 rows
    _quant_case(dev, 2, 65536, 4, 64, 4, 4, outliers=True)


@pytest.fixture(params=["matrix", "generic"])
def indexer_path(request):
    """Run a case on the matrix-core indexer (default) and again on the generic VALU indexer."""
    from aetherkv import _lib as L
    prev = L.lib().aekv_set_generic_kernels(1 if request.param == "generic" else 0)
    yield request.param
    L.lib().aekv_set_generic_kernels(prev)


@pytest.mark.parametrize("B,S,IH,IC,bits,k,valid,mode", [
    (2, 1, 4, 64, 4, 8, None, "softplus"),                         # one key, k > S: -1 padding
    (2, 100, 4, 64, 8, 256, [100, 17], "raw"),                     # k > visible keys
    (3, 20000, 16, 128, 4, 1024, [20000, 8193, 2049], "relu_w"),   # 4 row blocks, largest k
    (2, 9000, 3, 128, 8, 1, None, "softplus"),                     # heads not a multiple of 4, k = 1
    (2, 70000, 8, 64, 4, 512, [70000, 16385], "softplus"),         # many chunks, ragged tail
])
def test_quant_indexer_shapes_both_paths(dev, indexer_path, B, S, IH, IC, bits, k, valid, mode):
    _quant_case(dev, B, S, IH, IC, bits, 50 + S % 97, mode=mode, k=k, valid=valid)


def _equal_key_rows(dev, B, S, IH, IC, bits):
    """Every key the same code row (equal scores before the scales), queries with positive dots."""
    pq = PolarQuant(bits)
    row = normal((1, 1, IC), 5, dtype=torch.bfloat16)
    codes, scale = pq.encode(row.expand(B, S, IC).contiguous().to(dev))
    q = normal((B, IH, IC), 6, dtype=torch.float32)
    keyf = pq.decode(codes[:1, :1], scale[:1, :1], out_dtype=torch.float32).cpu()[0, 0]
    q = torch.where((q @ keyf)[..., None] < 0, -q, q).to(dev)   # positive dots: nonzero scores
    return pq, codes, scale, q, torch.ones(B, IH, device=dev)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n_special", [300, 100])
@pytest.mark.parametrize("S", [20000, 65536])
def test_quant_indexer_exact_ties_take_lowest_indices(dev, indexer_path, bits, n_special, S):
    # Every key is the same code row (equal scores); n_special keys get twice the scale (exactly
    # twice the score).  300 specials put the k-th key inside a small tied group; 100 specials
    # leave 156 picks among all the other, equal keys (the threshold bin overflows any candidate
    # list; at S = 65536 every one of the 4096 slots qualifies, more than the select's slot list
    # holds).
    B, IH, IC, k = 2, 4, 64, 256
    pq, codes, scale, q, w = _equal_key_rows(dev, B, S, IH, IC, bits)
    g = torch.Generator().manual_seed(9)
    special = [torch.randperm(S, generator=g)[:n_special].sort().values for _ in range(B)]
    scale = scale.clone()
    for b in range(B):
        scale[b, special[b].to(dev)] *= 2
    idx, sc = csa_indexer_topk_quant(q, w, codes, scale, k, quant=pq, return_scores=True)
    idx = idx.cpu()
    for b in range(B):
        sp = special[b]
        rest = torch.tensor(sorted(set(range(S)) - set(sp.tolist())), dtype=torch.int64)
        want = sp[:k] if n_special >= k else torch.cat([sp, rest[:k - n_special]])
        assert torch.equal(idx[b], want), (b, idx[b][:8], want[:8])
    # scores: specials exactly twice the others
    s = sc.cpu()
    top = min(n_special, k)
    assert torch.all(s[:, :top] == s[:, :1]) and torch.all(s[:, top:] * 2 == s[:, :1])


@pytest.mark.parametrize("S", [20000, 65536])
def test_quant_indexer_top_keys_spread_over_many_binades(dev, indexer_path, S):
    # 300 keys at random positions get scales spread over 12 binades (2^(1 + 12 i / 300) times the
    # common one, each a factor 1.028 apart); the top 256 of them are the answer, in scale order.
    # The k-th largest slot maximum then lies ~10 binades below the row's largest, further down
    # than the select's first, per-wave threshold search looks; its whole-histogram search finds it.
    B, IH, IC, k, n_sp = 2, 4, 64, 256, 300
    pq, codes, scale, q, w = _equal_key_rows(dev, B, S, IH, IC, 4)
    g = torch.Generator().manual_seed(13)
    mult = torch.tensor([2.0 ** (1 + 12 * i / n_sp) for i in range(n_sp)], dtype=torch.float32)
    scale = scale.clone()
    want = []
    for b in range(B):
        pos = torch.randperm(S, generator=g)[:n_sp]
        scale[b, pos.to(dev)] *= mult.to(dev)[:, None]
        want.append(pos.flip(0)[:k])   # largest multiplier first
    idx, sc = csa_indexer_topk_quant(q, w, codes, scale, k, quant=pq, return_scores=True)
    idx, sc = idx.cpu(), sc.cpu()
    for b in range(B):
        assert torch.equal(idx[b], want[b]), (b, idx[b][:8], want[b][:8])
        assert torch.all(sc[b, 1:] < sc[b, :-1])


def test_fp32_indexer_default_rule_is_the_reference_functions(dev):
    # an unchanged caller of csa_indexer_topk (no mode) gets the rule of the function it replaces:
    # sum over heads with w_h > 0 of w_h * (q_h . k), no relu on the dot
    # (aether_kernels/csrc/csa_indexer_cuda.cu:44-55; "relu applied internally", sparse_attention.py:57)
    B, S, IH, IC, k = 3, 3000, 4, 64, 256
    g = torch.Generator().manual_seed(91)
    q = torch.randn(B, IH, IC, generator=g)
    kv = torch.randn(B, S, IC, generator=g)
    w = torch.randn(B, IH, generator=g) * 2
    w[0] = torch.tensor([1.5, -0.5, 0.25, -2.0])   # mixed signs: relu on the weight matters
    idx = csa_indexer_topk(q.to(dev), kv.to(dev), w.to(dev), k).cpu().numpy()
    scores = O.index_scores(q.numpy(), w.numpy(), kv.numpy(), mode="relu_w")
    tol = score_error_bound(q.numpy(), w_act(w.numpy(), "relu_w"), kv.numpy())
    assert_topk_matches(idx, scores, k, tol)
    # the softplus rule selects a different set on these rows, so the default is not it
    soft = O.topk(O.index_scores(q.numpy(), w.numpy(), kv.numpy(), mode="softplus"), k)[0]
    assert any(set(idx[b]) != set(soft[b]) for b in range(B))


def _cfg5_index_inputs(dev, B=64, S=65536, IH=4, IC=64, seed=4):
    """cfg5's index cache and query: 4-bit keys, N(0,1) with 2% outlier channels x8 (seed 4)."""
    pq = PolarQuant(4)
    codes, scale = pq.encode(normal_with_outliers((B, S, IC), seed + 1000, device=dev, trailing_dims=1))
    q = normal((B, IH, IC), seed + 2, dtype=torch.float32).to(dev)
    w = normal((B, IH), seed + 3, dtype=torch.float32).to(dev)
    return pq, codes, scale, q, w


def _oracle_rows_check(pq, codes, scale, q, w, idx, k, rows, valid=None, mode="softplus"):
    """Oracle top-k check of the given rows, 8 rows at a time (keys dequantised in fp32)."""
    IC = q.shape[-1]
    dg = O.diag(42, IC)
    rows = list(rows)
    for i in range(0, len(rows), 8):
        r = rows[i:i + 8]
        keys = O.decode(codes[r].cpu().numpy(), scale[r].cpu().numpy(), pq.bits, dg, "f32")
        qn, wn = q[r].cpu().numpy(), w[r].cpu().numpy()
        vr = None if valid is None else np.asarray(valid)[r].astype(np.int32)
        scores = O.index_scores(qn, wn, keys, valid=vr, mode=mode)
        tol = score_error_bound(qn, w_act(wn, mode), keys, extra_rel=16 * math.log2(IC) * 2.0 ** -24)
        assert_topk_matches(idx[r], scores, k, tol, vr)


@pytest.mark.parametrize("ragged", [False, True])
def test_config5_indexer_all_rows_multi_group_waves(dev, ragged):
    # cfg5's whole launch: 64 rows x 65536 4-bit keys.  The score kernel gives each wave two slot groups
    # here (64 rows x 256 groups / 8192); 2-row launches give one.  Both must agree bit for bit, and every
    # row must match the oracle's exact top-k.  Ragged visible counts end a wave's keys part-way through
    # its groups.
    B, S, k = 64, 65536, 256
    pq, codes, scale, q, w = _cfg5_index_inputs(dev)
    valid = None
    if ragged:
        g = torch.Generator().manual_seed(45)
        valid = torch.randint(0, S + 1, (B,), generator=g, dtype=torch.int32)
        valid[:6] = torch.tensor([0, 1, 255, 256, 257, 65535], dtype=torch.int32)
        valid[6:12] = torch.tensor([300, 511, 513, 767, 1025, 33000], dtype=torch.int32)
    vd = None if valid is None else valid.to(dev)
    print(f"cfg5 indexer, all 64 rows, ragged={ragged}", flush=True)
    idx, sc = csa_indexer_topk_quant(q, w, codes, scale, k, quant=pq, valid=vd, return_scores=True)
    torch.cuda.synchronize()
    for b in range(0, B, 2):
        one, sc1 = csa_indexer_topk_quant(q[b:b + 2], w[b:b + 2], codes[b:b + 2], scale[b:b + 2], k, quant=pq,
                                          valid=None if vd is None else vd[b:b + 2], return_scores=True)
        assert torch.equal(idx[b:b + 2], one), f"rows {b}, {b + 1}: 64-row launch differs from a 2-row launch"
        assert torch.equal(sc[b:b + 2], sc1), f"rows {b}, {b + 1}: scores differ"
    rows = range(B) if not ragged else list(range(12)) + list(range(12, B, 7))
    _oracle_rows_check(pq, codes, scale, q, w, idx.cpu().numpy(), k, rows,
                       None if valid is None else valid.numpy())


def test_prefill_chunk_indexer_bench_shape(dev):
    # the CSA prefill chunk of the benchmark: 8 sequences x 256 targets at positions 65280..65535 over
    # 16384 8-bit blocks (top-256).  The score kernel shares each key group among 4 targets and gives
    # each wave 8 slot groups (512 row groups x 128 groups / 8192).  Sampled targets against the
    # single-target indexer bit for bit and against the oracle.
    from aetherkv.prefill import csa_prefill_indexer_topk_quant

    B, T, S, IH, IC, k = 8, 256, 16384, 4, 64, 256
    pq = PolarQuant(8)
    codes, scale = pq.encode(normal((B, S, IC), 12).to(dev))
    index_q = normal((B, T, IH, IC), 13, dtype=torch.float32).to(dev)
    index_w = normal((B, T, IH), 14, dtype=torch.float32).to(dev)
    pos = torch.arange(65280, 65536)
    valid = torch.clamp(torch.div(pos + 1, 4, rounding_mode="floor"), max=S).to(torch.int32)   # visible blocks
    print("prefill chunk indexer, 2048 rows", flush=True)
    idx = csa_prefill_indexer_topk_quant(index_q, index_w, codes, scale, k, quant=pq, valid=valid)
    torch.cuda.synchronize()
    dg = O.diag(42, IC)
    keys = O.decode(codes.cpu().numpy(), scale.cpu().numpy(), 8, dg, "f32")
    for t in (0, 1, 2, 3, 4, 127, 128, 200, 254, 255):
        vt = torch.full((B,), int(valid[t]), dtype=torch.int32)
        one = csa_indexer_topk_quant(index_q[:, t], index_w[:, t], codes, scale, k, quant=pq, valid=vt.to(dev))
        assert torch.equal(idx[:, t], one), f"target {t}"
        qn, wn = index_q[:, t].cpu().numpy(), index_w[:, t].cpu().numpy()
        scores = O.index_scores(qn, wn, keys, valid=vt.numpy())
        tol = score_error_bound(qn, w_act(wn, "softplus"), keys, extra_rel=16 * math.log2(IC) * 2.0 ** -24)
        assert_topk_matches(idx[:, t].cpu().numpy(), scores, k, tol, vt.numpy())
