"""Pins the oracle's TurboQuant rounding points against the reference's own torch op sequence (CPU).

The GPU codec tests compare bit for bit with oracle/aekv_oracle.c, so the oracle's fp32 rounding
points must be the reference's.  Two of them are invisible to dyadic known answers:

* the quantiser divides, then multiplies: ``rotated / max_abs * Q`` (two roundings,
  aether_2b/turbo_quant.py:153 and :159), not ``rotated * (Q / max_abs)``;
* decode scales the codes BEFORE the transform: ``q_f32 * scale_f32`` then ``_wht(rotated) * diag``
  (turbo_quant.py:191-203, :209), not ``_wht(q) * scale``.

Here the reference's sequence is written out in torch eager ops on the CPU, so torch's own kernels
do the rounding, and the oracle must equal it bit for bit on 2.3e5 rows: N(0,1), outlier-channel,
wide-range and near-tie rows, D in {64, 128}, bits in {4, 8}.  The same rows are shown to separate
the reference's orderings from the two alternatives above, and two known-answer rows whose expected
codes follow from exact rational arithmetic (each fp32 step rounded by hand) fail under either
alternative.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import scipy.linalg
import torch

import oracle as O
import torch_ref as T

N_ROWS = {64: 40000, 128: 75000}   # per (d, bits): 2 * (40000 + 75000) = 230000 rows in all


# ---- the reference's op sequence, torch eager (oracle/torch_ref.py) ---------------------------------
_t_wht = T.wht
_t_encode = T.encode
_t_unpack = T.unpack
_t_decode = T.decode


# ---- the two alternative orderings (used only to show the inputs separate them) --------------------
def _t_codes_mul_first(x: torch.Tensor, bits: int, diag: torch.Tensor) -> torch.Tensor:
    rot = _t_wht(x.float() * diag)
    q_max = 127.0 if bits == 8 else 7.0
    max_abs = rot.abs().amax(dim=-1, keepdim=True).clamp_(min=1e-8)
    return (rot * (q_max / max_abs)).round_().clamp_(-q_max, q_max)


def _t_decode_scale_after(data, scale, bits, diag, out_dtype):
    return (_t_wht(_t_unpack(data, bits)) * scale * diag).to(out_dtype)


# ---- inputs ------------------------------------------------------------------------------------------
def _rows(d: int, n: int, seed: int, diag: np.ndarray) -> torch.Tensor:
    """bf16 rows, four kinds in equal parts: N(0,1); 2% outlier channels x8; rows scaled by 2^U(-20,20);
    near-tie rows (rotated values placed ~1e-6 relative from the quantiser's half-integer boundaries
    of both widths, through the inverse transform)."""
    g = torch.Generator().manual_seed(seed)
    q = n // 4
    plain = torch.randn(q, d, generator=g)
    outl = torch.randn(q, d, generator=g)
    ch = torch.randperm(d, generator=g)[: max(1, round(0.02 * d))]
    outl[:, ch] *= 8.0
    wide = torch.randn(q, d, generator=g) * torch.exp2(torch.randint(-20, 21, (q, 1), generator=g).float())
    m = torch.rand(n - 3 * q, 1, generator=g, dtype=torch.float64) * 30 + 1
    q_max = torch.where(torch.rand(n - 3 * q, 1, generator=g) < 0.5, 7.0, 127.0).double()
    k = torch.randint(-7, 7, (n - 3 * q, d), generator=g).double()
    k = torch.where(q_max > 7, k * 9, k)
    target = (k + 0.5) / q_max * m * (1 + 1e-6 * torch.randn(n - 3 * q, d, generator=g, dtype=torch.float64))
    target[:, 0] = m[:, 0]                                    # the row's max sets max_abs = m
    h = torch.from_numpy(scipy.linalg.hadamard(d).astype(np.float64)) / d ** 0.5
    near = (target @ h.T) * torch.from_numpy(diag.astype(np.float64))
    return torch.cat([plain, outl, wide, near.float()]).to(torch.bfloat16)


def _bits_u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module", params=[(64, 4), (64, 8), (128, 4), (128, 8)], ids=lambda p: f"d{p[0]}-{p[1]}bit")
def case(request):
    d, bits = request.param
    dg = O.diag(42, d)
    x = _rows(d, N_ROWS[d], seed=1000 * d + bits, diag=dg)
    diag_t = torch.from_numpy(dg)
    data_t, scale_t = _t_encode(x, bits, diag_t)
    return dict(d=d, bits=bits, dg=dg, diag_t=diag_t, x=x, data_t=data_t, scale_t=scale_t)


def test_encode_equals_torch_op_sequence(case):
    codes, scale = O.encode(_bits_u16(case["x"]), "bf16", case["bits"], case["dg"])
    np.testing.assert_array_equal(scale, case["scale_t"].numpy())
    want = case["data_t"].numpy()
    assert codes.dtype == want.dtype
    np.testing.assert_array_equal(codes, want)


@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_decode_equals_torch_op_sequence(case, out):
    bits = case["bits"]
    got = O.decode(case["data_t"].numpy(), case["scale_t"].numpy(), bits, case["dg"], out)
    want = _t_decode(case["data_t"], case["scale_t"], bits, case["diag_t"],
                     torch.bfloat16 if out == "bf16" else torch.float32)
    np.testing.assert_array_equal(got, _bits_u16(want) if out == "bf16" else want.numpy())


def test_inputs_separate_the_quantiser_orderings(case):
    # rot * (Q / m) instead of rot / m * Q must change some codes on these rows, else the test above
    # could not tell the two apart.
    bits = case["bits"]
    ref = _t_unpack(case["data_t"], bits) if bits == 4 else case["data_t"].float()
    alt = _t_codes_mul_first(case["x"], bits, case["diag_t"])
    assert int((alt != ref).any(-1).sum()) > 0


def test_inputs_separate_the_decode_orderings(case):
    bits = case["bits"]
    ref = _t_decode(case["data_t"], case["scale_t"], bits, case["diag_t"], torch.bfloat16)
    alt = _t_decode_scale_after(case["data_t"], case["scale_t"], bits, case["diag_t"], torch.bfloat16)
    assert int((alt != ref).sum()) > 100


# ---- known answers from exact rational arithmetic ----------------------------------------------------
def _rn32(v: Fraction) -> Fraction:
    """Round a rational to the nearest fp32 (ties to even); normal range only."""
    if v == 0:
        return Fraction(0)
    s = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp = Fraction(2) ** (e - 23)
    n, r = divmod(a, ulp)
    if r > ulp / 2 or (r == ulp / 2 and n % 2 == 1):
        n += 1
    return s * n * ulp


def _rne_int(v: Fraction) -> int:
    n = v.numerator // v.denominator
    r = v - n
    return n + 1 if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1) else n


def _x_for_rotated(rot, dg) -> np.ndarray:
    """d = 4: x with _wht(x * diag) == rot exactly (integer rot, all sums exact in fp32)."""
    h = scipy.linalg.hadamard(4).astype(np.float64)
    return (dg * (0.5 * h @ np.asarray(rot, np.float64))).astype(np.float32)


def _find_quantiser_kat(q_max: int):
    """Smallest integer rot = [m, r, 0, 0] whose code of r differs between RN(RN(r/m)*Q) and
    RN(r*RN(Q/m)) after round-half-even, both computed exactly here."""
    for m in range(3, 4000):
        qm = _rn32(Fraction(q_max, m))
        for r in range(1, m):
            ref = _rne_int(_rn32(_rn32(Fraction(r, m)) * q_max))
            alt = _rne_int(_rn32(r * qm))
            if ref != alt:
                return m, r, ref, alt
    raise AssertionError("no separating row found")


@pytest.mark.parametrize("bits", [4, 8])
def test_quantiser_divide_then_multiply_known_answer(bits):
    q_max = 7 if bits == 4 else 127
    m, r, ref, alt = _find_quantiser_kat(q_max)
    dg = O.diag(42, 4)
    codes, scale = O.encode(_x_for_rotated([m, r, 0, 0], dg)[None], "f32", bits, dg)
    assert scale[0, 0] == np.float32(_rn32(Fraction(m, q_max)))
    if bits == 8:
        assert list(codes[0]) == [q_max, ref, 0, 0]
    else:
        assert list(codes[0]) == [(q_max & 15) | ((ref & 15) << 4), 0]
    assert ref != alt


def _decode_exact(codes, s: Fraction, dg):
    """Reference decode of a d = 4 int8 row with every fp32 step rounded by hand:
    rot = RN(c*s); h=1 and h=2 butterflies RN(a+b), RN(a-b); * fp32(0.5) (exact); * diag."""
    v = [_rn32(c * s) for c in codes]
    v = [_rn32(v[0] + v[1]), _rn32(v[0] - v[1]), _rn32(v[2] + v[3]), _rn32(v[2] - v[3])]
    v = [_rn32(v[0] + v[2]), _rn32(v[1] + v[3]), _rn32(v[0] - v[2]), _rn32(v[1] - v[3])]
    return [x / 2 * int(g) for x, g in zip(v, dg)]


def _decode_scale_after(codes, s: Fraction, dg):
    v = list(codes)
    v = [v[0] + v[1], v[0] - v[1], v[2] + v[3], v[2] - v[3]]
    v = [v[0] + v[2], v[1] + v[3], v[0] - v[2], v[1] - v[3]]
    return [_rn32(Fraction(x, 2) * s) * int(g) for x, g in zip(v, dg)]


def test_decode_scale_before_transform_known_answer():
    # Search small int8 rows and a non-dyadic fp32 scale for one where scaling before the butterflies
    # (the reference) and after them give different fp32 outputs; the oracle must give the former.
    dg = np.array([1, -1, -1, 1], np.float32)
    s = _rn32(Fraction(1, 3))                 # fp32(1/3): non-dyadic
    rng = np.random.default_rng(7)
    for _ in range(10000):
        c = [int(v) for v in rng.integers(-127, 128, 4)]
        ref = _decode_exact(c, s, dg)
        if ref != _decode_scale_after(c, s, dg):
            break
    else:
        raise AssertionError("no separating row found")
    got = O.decode(np.array([c], np.int8), np.array([[float(s)]], np.float32), 8, dg, "f32")
    np.testing.assert_array_equal(got[0], np.array([float(v) for v in ref], np.float32))


# ---- the torch CSA decode step (the CPU baseline) against the C oracle ---------------------------------
@pytest.mark.parametrize("bits", [4, 8])
def test_torch_csa_decode_step_matches_c_oracle(bits):
    # aether_2b/serving.py:597-625 as torch ops (oracle/torch_ref.py) and the C oracle's pieces must agree:
    # the selected set up to fp32 near-ties, the attention within the path's tolerance (fp32 compute)
    from topk_check import assert_topk_matches, score_error_bound

    B, S, H, D, W, IH, IC, k = 3, 700, 12, 128, 32, 4, 64, 64
    g = torch.Generator().manual_seed(bits)
    dk, di = torch.from_numpy(O.diag(42, D)), torch.from_numpy(O.diag(42, IC))
    kv_codes, kv_scale = T.encode(torch.randn(B, S, D, generator=g).to(torch.bfloat16), bits, dk)
    ix_codes, ix_scale = T.encode(torch.randn(B, S, IC, generator=g).to(torch.bfloat16), bits, di)
    q = torch.randn(B, 1, H, D, generator=g).to(torch.bfloat16)
    iq, iw = torch.randn(B, IH, IC, generator=g), torch.randn(B, IH, generator=g)
    win = torch.randn(B, W, D, generator=g).to(torch.bfloat16)
    sink = torch.randn(H, generator=g)
    out, idx = T.csa_decode_step(q, iq, iw, ix_codes, ix_scale, kv_codes, kv_scale, win, sink, bits, di, dk, k,
                                 compute_dtype=torch.float32)
    keys = O.decode(ix_codes.numpy(), ix_scale.numpy(), bits, O.diag(42, IC), "f32")
    scores = O.index_scores(iq.numpy(), iw.numpy(), keys)
    wa = np.log1p(np.exp(iw.numpy().astype(np.float64)))
    assert_topk_matches(idx.numpy(), scores, k,
                        score_error_bound(iq.numpy(), wa, keys, extra_rel=96 * 2.0 ** -24))
    want = O.quant_attention(q.float().numpy().reshape(B, H, D), kv_codes.numpy(), kv_scale.numpy(), idx.numpy(),
                             win.float().numpy(), sink.numpy(), O.diag(42, D), bits, D ** -0.5)
    np.testing.assert_allclose(out.float().numpy().reshape(B, H, D), want, rtol=1e-2, atol=2e-3)
