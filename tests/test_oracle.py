"""Pins for the CPU oracle (oracle/aekv_oracle.c) — runs on CPU, no GPU.

The reference's own tests hold no golden vectors for this path (only properties and tolerances,
tests/test_turbo_quant.py and tests/test_cuda_runtime.py in the reference).  Each oracle function is
pinned here by (a) hand-derived known answers that a plausible mistake (stage order, sign, rounding
mode, nibble order, sign extension) fails, (b) library routines (torch.Generator, scipy's Hadamard
matrix, numpy float64 brute force), and (c) the reference tests' own properties and thresholds.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import scipy.linalg
import torch

import oracle as O


# ---- Rademacher diagonal (turbo_quant.py:111-121) ------------------------------------------------
@pytest.mark.parametrize("seed", [42, 0, 7, 123456])
@pytest.mark.parametrize("d", [2, 8, 16, 64, 128, 256, 512])
def test_diag_matches_torch_generator(seed, d):
    g = torch.Generator()
    g.manual_seed(seed * 10007 + d)
    r = torch.rand(d, generator=g)
    want = torch.where(r > 0.5, torch.ones(d), -torch.ones(d)).numpy()
    np.testing.assert_array_equal(O.diag(seed, d), want)


def test_diag_differs_between_dims():
    # reference test_polar_quant_different_dims_use_different_diagonals
    assert not np.array_equal(O.diag(42, 128)[:64], O.diag(42, 64))


def test_wht_scale_constant():
    # fp32(128 ** -0.5) = 0x3DB504F3; powers of four are exact
    assert O.wht_scale(128).view(np.uint32) == 0x3DB504F3
    assert O.wht_scale(64) == np.float32(0.125)
    assert O.wht_scale(4) == np.float32(0.5)


def test_wht_final_scale_rounds_like_torch_scalar_multiply():
    # turbo_quant.py:76 multiplies an fp32 tensor by the Python double d ** -0.5.  torch rounds the
    # scalar to fp32 first; RN32(x * c_double) differs from RN32(x * fp32(c)) for ~20% of inputs, so
    # torch itself decides which one the oracle must do.  A scaled basis vector makes every butterfly
    # exact (one nonzero), leaving only the final multiply: every output is +-RN(v * c).
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(4096) * 37).astype(np.float32)
    c64 = 128 ** -0.5
    via_double = (v.astype(np.float64) * c64).astype(np.float32)
    torch_out = (torch.from_numpy(v) * c64).numpy()
    assert np.count_nonzero(torch_out != via_double) > 100   # the probe separates the two readings
    x = np.zeros((v.size, 128), np.float32)
    x[:, 0] = v
    got = O.wht(x)
    np.testing.assert_array_equal(got, np.repeat(torch_out[:, None], 128, axis=1))


def test_round_is_half_to_even_in_torch():
    # turbo_quant.py:152,158 use torch.round; the oracle's tie handling assumes half-to-even.
    t = torch.round(torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, 3.5, 6.5, -6.5]))
    np.testing.assert_array_equal(t.numpy(), [0, 2, 2, -0.0, -2, 4, 6, -6])


def test_decode_bf16_cast_matches_torch():
    # turbo_quant.py:211 `.to(out_dtype)`: the oracle's bf16 output must equal torch's RNE cast of
    # its own fp32 output, ties included.
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((512, 128)) * np.exp2(rng.integers(-6, 6, (512, 1)))).astype(np.float32)
    dg = O.diag(42, 128)
    codes, scale = O.encode(x, "f32", 8, dg)
    f32 = O.decode(codes, scale, 8, dg, "f32")
    bf = O.decode(codes, scale, 8, dg, "bf16")
    want = torch.from_numpy(f32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf, want)


# ---- WHT (turbo_quant.py:49-76) ------------------------------------------------------------------
def test_wht_stage_order_known_answer():
    # Stages run h=1 then h=2 with fp32 rounding at each add:
    #   h=1: [RN(2^24+1)=2^24, 2^24-1, 1, 1];  h=2: [RN(2^24+1)=2^24, 2^24, 2^24-1, 2^24-2];  *0.5
    # The reversed order would give [2^23, 2^23-0.5, 2^23, 2^23-1]; exact math [2^23+1, 2^23, 2^23, 2^23-1].
    x = np.array([[2.0 ** 24, 1.0, 1.0, 0.0]], dtype=np.float32)
    np.testing.assert_array_equal(O.wht(x)[0], np.array([2 ** 23, 2 ** 23, 2 ** 23 - 0.5, 2 ** 23 - 1], np.float32))


def test_wht_sum_difference_layout_known_answer():
    # d=2: [a+b, a-b] * fp32(2^-0.5)
    c = np.float32(2.0 ** -0.5)
    np.testing.assert_array_equal(O.wht(np.array([[3.0, 1.0]], np.float32))[0], np.array([4, 2], np.float32) * c)


@pytest.mark.parametrize("d", [2, 4, 16, 64, 128, 512])
def test_wht_matches_sylvester_hadamard(d):
    rng = np.random.default_rng(d)
    x = rng.standard_normal((8, d)).astype(np.float32)
    want = x.astype(np.float64) @ scipy.linalg.hadamard(d).T.astype(np.float64) / math.sqrt(d)
    got = O.wht(x).astype(np.float64)
    # log2(d) fp32 stages: |err| <= (log2 d + 1) * 2^-24 * sum|x| / sqrt(d) (loose)
    bound = (math.log2(d) + 2) * 2.0 ** -24 * np.abs(x).sum(axis=1, keepdims=True) / math.sqrt(d) * 4
    assert np.all(np.abs(got - want) <= bound)


def test_wht_self_inverse():
    rng = np.random.default_rng(0)
    for d in (64, 128):
        x = rng.standard_normal((4, 16, d)).astype(np.float32)
        np.testing.assert_allclose(O.wht(O.wht(x)), x, atol=1e-5)


def test_wht_rejects_non_power_of_two():
    with pytest.raises(ValueError, match="power of 2"):
        O.wht(np.zeros((3, 12), np.float32))


# ---- encode / decode (turbo_quant.py:127-211) -----------------------------------------------------
def _x_for_rotated(rot: np.ndarray, dg: np.ndarray) -> np.ndarray:
    """x with _wht(x * diag) == rot exactly for d = 4 (c = 0.5, small dyadic values)."""
    h = scipy.linalg.hadamard(4).astype(np.float64)
    return (dg * (0.5 * h @ rot.astype(np.float64))).astype(np.float32)


def test_encode4_known_answer_half_to_even_and_nibbles():
    # rot = [14, 1, 3, 5]: m = 14, scale = 2, rot/m*7 = [7, 0.5, 1.5, 2.5] exactly (RN(RN(k/14)*7) = k/2)
    # round half to even -> [7, 0, 2, 2]; bytes: (7 | 0<<4) = 0x07, (2 | 2<<4) = 0x22.
    dg = O.diag(42, 4)
    x = O.f32_to_bf16(_x_for_rotated(np.array([14, 1, 3, 5]), dg))[None]
    codes, scale = O.encode(x, "bf16", 4, dg)
    assert codes.dtype == np.uint8 and codes.shape == (1, 2) and scale.shape == (1, 1)
    np.testing.assert_array_equal(codes[0], [0x07, 0x22])
    assert scale[0, 0] == np.float32(2.0)


def test_encode4_negative_codes_twos_complement():
    # rot = [-14, -7, 7, 0]: q = [-7, -3.5 -> -4, 3.5 -> 4, 0]; -7 & 15 = 0x9, -4 & 15 = 0xC
    dg = O.diag(42, 4)
    x = _x_for_rotated(np.array([-14, -7, 7, 0]), dg)[None]
    codes, scale = O.encode(x, "f32", 4, dg)
    np.testing.assert_array_equal(codes[0], [0x09 | (0x0C << 4), 0x04])
    assert scale[0, 0] == np.float32(2.0)


def test_encode8_known_answer_ties():
    # rot = [254, 1, 3, 5]: rot/m*127 = [127, 0.5, 1.5, 2.5] exactly -> [127, 0, 2, 2] (half to even)
    dg = O.diag(42, 4)
    x = _x_for_rotated(np.array([254, 1, 3, 5]), dg)[None]
    codes, scale = O.encode(x, "f32", 8, dg)
    assert codes.dtype == np.int8
    np.testing.assert_array_equal(codes[0], [127, 0, 2, 2])
    assert scale[0, 0] == np.float32(254.0) / np.float32(127.0)


def test_encode_zero_row_uses_eps_scale():
    dg = O.diag(42, 128)
    for bits, q in ((8, 127.0), (4, 7.0)):
        codes, scale = O.encode(np.zeros((2, 128), np.float32), "f32", bits, dg)
        assert not codes.any()
        assert scale[0, 0] == np.float32(np.float32(1e-8) / np.float32(q))


def test_decode4_known_answer_sign_extension():
    # byte 0x8F: low nibble 0xF -> -1 (even), high nibble 0x8 -> -8 (odd)
    # rot = [-1, -8, 0, 0] -> h=1 [-9, 7, 0, 0] -> h=2 [-9, 7, -9, 7] -> *0.5
    out = O.decode(np.array([[0x8F, 0x00]], np.uint8), np.array([[1.0]], np.float32), 4, np.ones(4, np.float32), "f32")
    np.testing.assert_array_equal(out[0], [-4.5, 3.5, -4.5, 3.5])


def test_decode4_known_answer_diag_and_scale():
    # codes [7,0,2,2] * 2 = [14,0,4,4] -> h=1 [14,14,8,0] -> h=2 [22,14,6,14] -> *0.5 -> * diag
    dg = np.array([1, -1, 1, -1], np.float32)
    out = O.decode(np.array([[0x07, 0x22]], np.uint8), np.array([[2.0]], np.float32), 4, dg, "f32")
    np.testing.assert_array_equal(out[0], [11, -7, 3, -7])


def test_decode8_known_answer():
    # codes [-127, 1] * 0.5 = [-63.5, 0.5] -> [-63, -64] * 2^-0.5 (fp32) -> * diag
    c = np.float32(2.0 ** -0.5)
    out = O.decode(np.array([[-127, 1]], np.int8), np.array([[0.5]], np.float32), 8, np.array([1, -1], np.float32), "f32")
    np.testing.assert_array_equal(out[0], [np.float32(-63) * c, -(np.float32(-64) * c)])


def test_bf16_rounding_is_rne():
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7 -> even (1.0); 1 + 3*2^-8 -> 1 + 2^-6 (even)
    vals = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8)], np.float32)
    np.testing.assert_array_equal(O.bf16_to_f32(O.f32_to_bf16(vals)), [1.0, 1 + 2 ** -6, -1.0])


@pytest.mark.parametrize("bits,thresh", [(8, 0.999), (4, 0.99)])
@pytest.mark.parametrize("d", [128, 64])
def test_roundtrip_cosine_reference_thresholds(bits, thresh, d):
    # thresholds of the reference's test_polar_quant_{8,4}bit_roundtrip
    torch.manual_seed(42)
    x = torch.randn(1, 64, d, dtype=torch.bfloat16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    dg = O.diag(42, d)
    codes, scale = O.encode(xb, "bf16", bits, dg)
    assert codes.shape == ((1, 64, d) if bits == 8 else (1, 64, d // 2))
    rec = O.bf16_to_f32(O.decode(codes, scale, bits, dg, "bf16"))
    xf = O.bf16_to_f32(xb)
    cos = (xf * rec).sum(-1) / np.linalg.norm(xf, axis=-1) / np.linalg.norm(rec, axis=-1)
    assert cos.mean() > thresh


def test_structured_input_thresholds():
    # reference test_polar_quant_{8,4}bit_structured_input
    torch.manual_seed(0)
    x = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    x[:, :, 0] = 10.0
    x += 0.01 * torch.randn_like(x)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    dg = O.diag(42, 128)
    xf = O.bf16_to_f32(xb)
    for bits, thresh in ((8, 0.999), (4, 0.95)):
        codes, scale = O.encode(xb, "bf16", bits, dg)
        rec = O.bf16_to_f32(O.decode(codes, scale, bits, dg, "bf16"))
        cos = (xf * rec).sum(-1) / np.linalg.norm(xf, axis=-1) / np.linalg.norm(rec, axis=-1)
        assert cos.mean() > thresh


def test_encode_invariants_random():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((256, 128)).astype(np.float32) * 3
    dg = O.diag(42, 128)
    rot = O.wht(x * dg)
    m = np.maximum(np.abs(rot).max(-1), np.float32(1e-8))
    for bits, q in ((8, 127), (4, 7)):
        codes, scale = O.encode(x, "f32", bits, dg)
        np.testing.assert_array_equal(scale[:, 0], m / np.float32(q))
        if bits == 8:
            assert np.abs(codes.astype(int)).max() <= 127
            assert np.all(np.abs(codes.astype(int)).max(-1) == 127)   # the max element maps to +-127
        else:
            nib = np.stack([codes & 15, codes >> 4], -1).reshape(256, 128).astype(int)
            nib = np.where(nib >= 8, nib - 16, nib)
            assert np.abs(nib).max() <= 7 and np.all(np.abs(nib).max(-1) == 7)


def test_encode_decode_deterministic_and_threads_agree():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1000, 128)).astype(np.float32)
    dg = O.diag(42, 128)
    a = O.encode(x, "f32", 4, dg, threads=1)
    b = O.encode(x, "f32", 4, dg, threads=8)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


# ---- indexer (modeling.py:609-616, serving.py:618-621, csa_indexer_cuda.cu:44-55) ----------------
def _brute_scores(q, w, keys, mode):
    dots = np.einsum("bhc,bsc->bhs", q.astype(np.float64), keys.astype(np.float64))
    w = w.astype(np.float64)
    if mode == "softplus":
        wa = np.where(w > 20, w, np.log1p(np.exp(np.minimum(w, 20))))
        return (np.maximum(dots, 0) * wa[..., None]).sum(1)
    if mode == "raw":
        return (np.maximum(dots, 0) * w[..., None]).sum(1)
    return (dots * np.maximum(w, 0)[..., None]).sum(1)


@pytest.mark.parametrize("mode", ["softplus", "raw", "relu_w"])
def test_index_scores_match_brute_force(mode):
    rng = np.random.default_rng(11)
    q = rng.standard_normal((3, 4, 16)).astype(np.float32)
    w = rng.standard_normal((3, 4)).astype(np.float32) * 3
    keys = rng.standard_normal((3, 50, 16)).astype(np.float32)
    np.testing.assert_allclose(O.index_scores(q, w, keys, mode=mode), _brute_scores(q, w, keys, mode), rtol=1e-12,
                               atol=1e-12)


def test_softplus_threshold():
    assert O.softplus(25.0) == 25.0
    assert abs(O.softplus(0.0) - math.log(2.0)) < 1e-15


def test_index_scores_valid_mask():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((2, 2, 8)).astype(np.float32)
    w = rng.standard_normal((2, 2)).astype(np.float32)
    keys = rng.standard_normal((2, 10, 8)).astype(np.float32)
    s = O.index_scores(q, w, keys, valid=np.array([10, 4], np.int32))
    assert np.isfinite(s[0]).all() and np.isneginf(s[1, 4:]).all() and np.isfinite(s[1, :4]).all()


def test_topk_order_ties_and_padding():
    s = np.array([[1.0, 3.0, 3.0, 2.0, 3.0], [5.0, 4.0, 0.0, 0.0, 0.0]])
    idx, sc = O.topk(s, 4, valid=np.array([5, 2], np.int32))
    np.testing.assert_array_equal(idx[0], [1, 2, 4, 3])      # score desc, index asc on ties
    np.testing.assert_array_equal(idx[1], [0, 1, -1, -1])    # fewer valid than k -> -1 padding
    ref = np.lexsort((np.arange(5), -s[0]))[:4]
    np.testing.assert_array_equal(idx[0], ref)


def test_topk_k_ge_visible_returns_all():
    rng = np.random.default_rng(2)
    s = rng.standard_normal((2, 7))
    idx, _ = O.topk(s, 7)
    for b in range(2):
        assert sorted(idx[b].tolist()) == list(range(7))


# ---- attention (aether_pipeline/serving.py:99-143; modeling.py:158-178) ---------------------------
def _brute_attention(q, kv, idx, sink, scale):
    B, T, H, D = q.shape
    S = kv.shape[1]
    out = np.zeros_like(q, dtype=np.float64)
    for b in range(B):
        for t in range(T):
            ok = [j for j in idx[b, t] if 0 <= j < S]
            K = kv[b, ok, 0].astype(np.float64)
            V = kv[b, ok, 1].astype(np.float64)
            for h in range(H):
                sk = float(sink if np.ndim(sink) == 0 or np.size(sink) == 1 else sink[h])
                lg = K @ q[b, t, h].astype(np.float64) * scale
                m = max(lg.max() if len(ok) else -np.inf, sk)
                e = np.exp(lg - m)
                out[b, t, h] = (e @ V) / (e.sum() + math.exp(sk - m))
    return out


def test_sink_attention_matches_brute_force_reference_shapes():
    # the reference's tests/test_cuda_runtime.py case: q [2,5,4,16], kv [2,23,2,16], topk [2,5,7]
    torch.manual_seed(0)
    q = torch.randn(2, 5, 4, 16).numpy()
    kv = torch.randn(2, 23, 2, 16).numpy()
    idx = torch.randint(0, 23, (2, 5, 7)).numpy()
    sink = torch.randn(4).numpy()
    got = O.sink_attention(q, kv, idx, sink, 0.125)
    np.testing.assert_allclose(got, _brute_attention(q, kv, idx, sink, 0.125), rtol=1e-6, atol=1e-7)


def test_sink_attention_skips_out_of_range_and_counts_duplicates():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 1, 2, 8)).astype(np.float32)
    kv = rng.standard_normal((1, 6, 2, 8)).astype(np.float32)
    idx = np.array([[[0, 3, 3, -1, 6, 99]]])
    got = O.sink_attention(q, kv, idx, np.array([0.3, -0.2], np.float32), 0.5)
    np.testing.assert_allclose(got, _brute_attention(q, kv, idx, np.array([0.3, -0.2]), 0.5), rtol=1e-6, atol=1e-7)


def test_sink_minus_inf_is_plain_softmax_attention():
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 1, 1, 8)).astype(np.float32)
    kv = rng.standard_normal((1, 5, 2, 8)).astype(np.float32)
    idx = np.arange(5)[None, None]
    got = O.sink_attention(q, kv, idx, np.array([-np.inf], np.float32), 0.7)[0, 0, 0]
    lg = kv[0, :, 0].astype(np.float64) @ q[0, 0, 0].astype(np.float64) * 0.7
    p = scipy.special.softmax(lg)
    np.testing.assert_allclose(got, p @ kv[0, :, 1].astype(np.float64), rtol=1e-6, atol=1e-7)


def test_sink_attention_no_valid_index_gives_zero():
    q = np.ones((1, 1, 1, 4), np.float32)
    kv = np.ones((1, 2, 2, 4), np.float32)
    got = O.sink_attention(q, kv, np.array([[[-1, 5]]]), np.array([0.0], np.float32), 1.0)
    assert not got.any()


def test_sink_attention_no_valid_index_and_sink_minus_inf_gives_zero_not_nan():
    # sparse_sink_attention_cuda.cu:102-113 sums weight * V over in-range indices only: with none
    # the output is 0 even though its normaliser e^{sink - max} is NaN at sink = max = -inf.  A
    # target with a valid index is unaffected (plain softmax, checked against brute force).
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 2, 2, 8)).astype(np.float32)
    kv = rng.standard_normal((1, 4, 2, 8)).astype(np.float32)
    idx = np.array([[[-1, 9, 4], [0, 2, -3]]])
    sink = np.array([-np.inf, -np.inf], np.float32)
    got = O.sink_attention(q, kv, idx, sink, 0.5)
    assert np.isfinite(got).all() and not got[0, 0].any()
    np.testing.assert_allclose(got[0, 1], _brute_attention(q[:, 1:], kv, idx[:, 1:], sink, 0.5)[0, 0],
                               rtol=1e-6, atol=1e-7)
    # the quantised decode attention: a row with no selected block and no window is 0 as well
    B, H, D, S = 2, 2, 16, 6
    dg = O.diag(42, D)
    codes, scale = O.encode(O.f32_to_bf16(rng.standard_normal((B, S, D)).astype(np.float32)), "bf16", 8, dg)
    qq = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((B, H, D)).astype(np.float32)))
    sel = np.array([[0, 3], [-1, -1]])
    out = O.quant_attention(qq, codes, scale, sel, np.zeros((B, 0, D), np.float32), np.full(H, -np.inf, np.float32),
                            dg, 8, 0.25)
    assert np.isfinite(out).all() and not out[1].any() and out[0].any()


@pytest.mark.parametrize("bits", [8, 4])
def test_quant_attention_equals_decode_gather_concat_attend(bits):
    # aether_2b/serving.py:597-625 composed from oracle pieces: decode to bf16, gather, concat window,
    # K = V, sink attention with full indices.
    rng = np.random.default_rng(8)
    B, H, D, S, K, W = 2, 3, 16, 20, 5, 4
    dg = O.diag(42, D)
    blocks = O.f32_to_bf16(rng.standard_normal((B, S, D)).astype(np.float32))
    codes, scale = O.encode(blocks, "bf16", bits, dg)
    q = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((B, H, D)).astype(np.float32)))
    win = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((B, W, D)).astype(np.float32)))
    sel = rng.integers(0, S, (B, K))
    sel[1, 2] = -1
    sink = rng.standard_normal(H).astype(np.float32)
    got = O.quant_attention(q, codes, scale, sel, win, sink, dg, bits, 0.25)
    dec = O.bf16_to_f32(O.decode(codes, scale, bits, dg, "bf16"))
    for b in range(B):
        src = np.concatenate([np.stack([dec[b, s] if s >= 0 else np.zeros(D, np.float32) for s in sel[b]]), win[b]])
        kv = np.stack([src, src], 1)[None]
        idx = np.array([[list(sel[b] >= 0) and [j if (j >= K or sel[b, j] >= 0) else -1 for j in range(K + W)]]])
        want = O.sink_attention(q[b][None, None], kv, idx, sink, 0.25)[0, 0]
        np.testing.assert_allclose(got[b], want, rtol=1e-6, atol=1e-7)
    # HCA: sel = None attends every block
    got_all = O.quant_attention(q, codes, scale, None, win, sink, dg, bits, 0.25)
    for b in range(B):
        src = np.concatenate([dec[b], win[b]])
        kv = np.stack([src, src], 1)[None]
        want = O.sink_attention(q[b][None, None], kv, np.arange(S + W)[None, None], sink, 0.25)[0, 0]
        np.testing.assert_allclose(got_all[b], want, rtol=1e-6, atol=1e-7)


def test_hca_compress_matches_softmax_weighted_sum():
    rng = np.random.default_rng(9)
    c = rng.standard_normal((2, 128, 16)).astype(np.float32)
    z = rng.standard_normal((2, 128, 16)).astype(np.float32) * 2
    w = scipy.special.softmax(z.astype(np.float64), axis=1)
    np.testing.assert_allclose(O.hca_compress(c, z), (w * c).sum(1), rtol=1e-6, atol=1e-7)


# ---- block emission (serving.py:495-505 _hca_emit, :557-576 _emit_csa_block) ---------------------

def _bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _torch_emit(c, z, bias, rope_dim, pos, inv_freq, norm_w, eps):
    """The engine's op sequence in torch (CPU): softmax(z.float()) -> bf16 weights -> (w * c).sum
    -> apply_rope(config=None shape) -> F.rms_norm; bf16 tensors as in the engine."""
    import torch.nn.functional as F
    zz = z if bias is None else z + bias
    w = torch.softmax(zz.float(), dim=1).to(c.dtype)
    comp = (w * c).sum(dim=1, keepdim=True)
    if rope_dim:
        B = comp.size(0)
        pp, rp = comp[..., :-rope_dim], comp[..., -rope_dim:]
        ang = pos.float().unsqueeze(-1) * inv_freq
        cos = torch.repeat_interleave(ang.cos(), 2, dim=-1).to(comp.dtype).view(B, 1, rope_dim)
        sin = torch.repeat_interleave(ang.sin(), 2, dim=-1).to(comp.dtype).view(B, 1, rope_dim)
        x1, x2 = rp[..., ::2], rp[..., 1::2]
        rot = torch.stack((-x2, x1), dim=-1).flatten(-2)
        comp = torch.cat([pp, rp * cos + rot * sin], dim=-1)
    if norm_w is not None:
        comp = F.rms_norm(comp, (comp.size(-1),), norm_w.to(comp.dtype), eps)
    return comp.squeeze(1)


@pytest.mark.parametrize("case", ["hca", "csa_main_first", "csa_main", "csa_index"])
def test_emit_block_matches_torch_op_sequence(case):
    g = torch.Generator().manual_seed({"hca": 1, "csa_main_first": 2, "csa_main": 3, "csa_index": 4}[case])
    B, m = 5, 128
    D = 64 if case == "csa_index" else 128
    L = m if case == "hca" else 2 * m
    c = torch.randn(B, L, D, generator=g).to(torch.bfloat16)
    z = (torch.randn(B, L, D, generator=g) * 2).to(torch.bfloat16)
    bias = None if case == "hca" else (torch.randn(L, D, generator=g) * 0.5).to(torch.bfloat16)
    if case == "csa_main_first":  # first CSA block: prev_b_c = 0, prev_b_z = -inf (serving.py:548-552)
        c[:, m:] = 0
        z[:, m:] = float("-inf")
    rope = 0 if case == "csa_index" else 64
    pos = torch.tensor([0, 127, 4095, 65535, 262143][:B], dtype=torch.int64)
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    nw = None if case == "csa_index" else (torch.rand(D, generator=g) * 2).to(torch.bfloat16)
    want = _torch_emit(c, z, bias, rope, pos, inv, nw, 1e-6)
    got = O.emit_block(_bits16(c), _bits16(z), None if bias is None else _bits16(bias), rope,
                       pos.numpy() if rope else None, inv.numpy() if rope else None,
                       None if nw is None else _bits16(nw), 1e-6)
    # libm exp/cos/sin and the order of the RMS sum may move an fp32 value by an ulp before a bf16
    # rounding: allow one bf16 ulp (same sign), and require nearly all bits equal
    w16 = _bits16(want).astype(np.int32)
    g16 = got.astype(np.int32)
    assert np.all(np.abs(g16 - w16) <= 1)
    assert np.mean(g16 == w16) > 0.995


def test_emit_block_pooling_reduces_to_hca_compress_and_plain_values():
    # no RoPE / norm: the pooled value is the softmax-weighted sum (hca_compress in exact math) up to
    # the bf16 roundings; one entry (L = 1) gives back c exactly
    g = torch.Generator().manual_seed(3)
    c = torch.randn(3, 128, 64, generator=g).to(torch.bfloat16)
    z = torch.randn(3, 128, 64, generator=g).to(torch.bfloat16)
    got = O.emit_block(_bits16(c), _bits16(z))
    gf = torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).float().numpy()
    exact = O.hca_compress(c.float().numpy(), z.float().numpy())
    np.testing.assert_allclose(gf, exact, rtol=2e-2, atol=2e-3)
    one = O.emit_block(_bits16(c[:, :1]), _bits16(z[:, :1]))
    np.testing.assert_array_equal(one, _bits16(c[:, 0]))


def test_diag_signs_match_the_committed_fixture():
    """The d = 64 and d = 128 diagonals of the engine's seed, frozen in tests/golden (written by
    tests/golden/make_diag_signs.py from torch's CPU generator, as turbo_quant.py:111-121 draws them):
    the oracle's MT19937 restatement and the library's host generator both reproduce them."""
    import json
    import ctypes
    from pathlib import Path

    import aetherkv._lib as L

    fx = json.loads((Path(__file__).parent / "golden" / "diag_signs_seed42.json").read_text())
    for d in (64, 128):
        want = np.array([1.0 if c == "+" else -1.0 for c in fx["signs"][str(d)]], np.float32)
        np.testing.assert_array_equal(O.diag(fx["seed"], d), want)
        host = np.empty(d, np.float32)
        assert L.lib().aekv_tq_diag(fx["seed"], d, host.ctypes.data_as(ctypes.c_void_p)) == L.OK
        np.testing.assert_array_equal(host, want)
