"""GPU parity of the TurboQuant codec: libaetherkv on the device vs the oracle on identical bytes.

Bar: codes, scales, WHT outputs and decoded values are bit-exact (turbo_quant.py:49-211).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from aetherkv import PolarQuant, _wht
from aetherkv.synthetic import normal_with_outliers
from conftest import bf16_bits

pytestmark = pytest.mark.gpu

TDT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def host_bits(t: torch.Tensor, name: str) -> np.ndarray:
    return t.cpu().numpy() if name == "f32" else bf16_bits(t)


def special_rows(n: int, d: int, dtype) -> torch.Tensor:
    """Random rows plus edge rows: zeros, a one-hot, denormal-range values, large values."""
    g = torch.Generator().manual_seed(1234 + d)
    x = torch.randn(n, d, generator=g) * 2
    x[0] = 0
    x[1] = 0
    x[1, d // 2] = -3.0
    x[2] = torch.randn(d, generator=g) * 1e-39
    x[3] = torch.randn(d, generator=g) * 1e3
    x[4] = 1.0
    return x.to(dtype)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("d", [2, 4, 8, 16, 32, 64, 128, 256, 512])
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_encode_bit_exact(dev, bits, d, dt):
    n = 1001  # not a multiple of the vectors handled per wave
    x = special_rows(n, d, TDT[dt])
    pq = PolarQuant(bits)
    codes, scale = pq.encode(x.to(dev))
    want_c, want_s = O.encode(host_bits(x, dt), dt, bits, O.diag(42, d))
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)
    np.testing.assert_array_equal(scale.cpu().numpy(), want_s)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("d", [2, 16, 64, 128, 512])
@pytest.mark.parametrize("odt", ["bf16", "f16", "f32"])
def test_decode_bit_exact(dev, bits, d, odt):
    rng = np.random.default_rng(d * 7 + bits)
    n = 777
    if bits == 8:
        codes = rng.integers(-127, 128, (n, d)).astype(np.int8)
    else:
        codes = rng.integers(0, 256, (n, d // 2)).astype(np.uint8)  # includes nibble 8 (-8)
    scale = (rng.random((n, 1)) * 0.5 + 1e-3).astype(np.float32)
    scale[0] = np.float32(1e-8) / np.float32(7)
    pq = PolarQuant(bits)
    out = pq.decode(torch.from_numpy(codes).to(dev), torch.from_numpy(scale).to(dev), out_dtype=TDT[odt])
    want = O.decode(codes, scale, bits, O.diag(42, d), odt)
    got = out.cpu().numpy() if odt == "f32" else bf16_bits(out)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("d", [1, 2, 8, 64, 128, 512])
@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_wht_bit_exact(dev, d, dt):
    x = special_rows(300, d, TDT[dt]) if d >= 8 else torch.randn(300, d).to(TDT[dt])
    got = _wht(x.to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, O.wht(host_bits(x, dt), dt))
    # self-inverse on the N(0,1) rows (reference test_wht_self_inverse: randn, atol 1e-5)
    if dt == "f32":
        xs = x[5:]
        np.testing.assert_allclose(_wht(_wht(xs.to(dev))).cpu().numpy(), xs.numpy(), atol=1e-5)


def test_config1_8bit_round_trip_bit_exact(dev):
    # benchmark configuration cfg1: [4096, 12, 128] bf16, N(0,1) with 2% outlier channels x8, seed 0, 8-bit
    x = normal_with_outliers((4096, 12, 128), 0)
    pq = PolarQuant(8)
    codes, scale = pq.encode(x.to(dev))
    assert codes.dtype == torch.int8 and codes.shape == (4096, 12, 128) and scale.shape == (4096, 12, 1)
    dg = O.diag(42, 128)
    want_c, want_s = O.encode(bf16_bits(x), "bf16", 8, dg)
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)
    np.testing.assert_array_equal(scale.cpu().numpy(), want_s)
    rec = pq.decode(codes, scale)
    assert rec.dtype == torch.bfloat16 and rec.shape == x.shape
    np.testing.assert_array_equal(bf16_bits(rec), O.decode(want_c, want_s, 8, dg, "bf16"))


def test_config2_4bit_full_layer_properties(dev):
    # benchmark configuration cfg2: 262144 x 1536 bf16 (12 heads x 128), 2% outliers x8, seed 1, 4-bit.
    T, H, D = 262144, 12, 128
    x = normal_with_outliers((T, H, D), 1, device=dev)
    pq = PolarQuant(4)
    codes, scale = pq.encode(x)
    codes2, scale2 = pq.encode(x)
    assert torch.equal(codes, codes2) and torch.equal(scale, scale2)  # deterministic
    assert codes.shape == (T, H, 64) and scale.shape == (T, H, 1)
    lo = (codes & 15).to(torch.int16)
    hi = (codes >> 4).to(torch.int16)
    assert not bool(((lo == 8) | (hi == 8)).any())                    # range [-7, 7], -8 never produced
    sx = lambda v: torch.where(v >= 8, v - 16, v)
    rowmax = torch.maximum(sx(lo).abs().amax(-1), sx(hi).abs().amax(-1))
    assert bool((rowmax == 7).all())                                  # the max element maps to +-7
    # bit-exact over the whole layer (the oracle's OpenMP encode takes well under a second)
    dg = O.diag(42, D)
    want_c, want_s = O.encode(bf16_bits(x), "bf16", 4, dg)
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)
    np.testing.assert_array_equal(scale.cpu().numpy(), want_s)
    rec = pq.decode(codes, scale)
    rows = torch.cat([torch.arange(0, 2048), torch.arange(2048, T, 977)]).to(dev)
    np.testing.assert_array_equal(bf16_bits(rec[rows]), O.decode(want_c[rows.cpu().numpy()], want_s[rows.cpu().numpy()], 4, dg, "bf16"))
    del want_c, want_s
    # quality: reference 4-bit threshold (cosine > 0.99 on Gaussian rows)
    cos = torch.nn.functional.cosine_similarity(x.float().view(-1, D), rec.float().view(-1, D), dim=-1)
    assert float(cos.mean()) > 0.99


def near_tie_rows(n: int, seed: int, d: int = 128) -> torch.Tensor:
    """bf16 rows whose rotated values sit on or next to quantiser ties: x*diag = a*e_0 + b*e_j gives
    raw butterflies a +- b, so raw/max*Q hits k + 1/2 for (a+b, a-b) = (14, 1), (14, 3) at Q = 7 and
    (254, 1), (254, 3), (254, 5) at Q = 127 ..."""
    g = torch.Generator().manual_seed(seed)
    dg = torch.from_numpy(O.diag(42, d))
    x = torch.zeros(n, d)
    pairs = [(7.5, 6.5), (8.5, 5.5), (9.5, 4.5), (127.5, 126.5), (3.5, 3.0), (1.0, 0.0), (0.75, 0.25), (128.5, 125.5),
             (129.5, 124.5)]
    for i in range(n):
        a, b = pairs[i % len(pairs)]
        j = int(torch.randint(1, d, (1,), generator=g))
        s = float(torch.randn(1, generator=g).sign())
        x[i, 0] = a * s
        x[i, j] = b * s * (1 if i % 2 else -1)
        if i % 3 == 0:
            x[i, (j + 5) % (d - 1) + 1] += 0.5
    return (x * dg).to(torch.bfloat16)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("d", [64, 128])
def test_encode_near_tie_rows_bit_exact(dev, bits, d):
    x = near_tie_rows(4001, 17, d)
    want_c, want_s = O.encode(bf16_bits(x), "bf16", bits, O.diag(42, d))
    pq = PolarQuant(bits)
    codes, scale = pq.encode(x.to(dev))
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)
    np.testing.assert_array_equal(scale.cpu().numpy(), want_s)


def wide_pair_rows(n: int, seed: int, d: int = 128) -> torch.Tensor:
    """bf16 rows whose only nonzero elements are one pair (2k, 2k+1) with magnitudes 2^9 .. 2^30
    apart: the first butterfly stage a +- b is then inexact in fp32 (ties included) and its rounding
    reaches the row maximum, i.e. the scale."""
    g = torch.Generator().manual_seed(seed)
    x = torch.zeros(n, d)
    k = torch.randint(0, d // 2, (n,), generator=g)
    ma = 1 + torch.randint(0, 128, (n,), generator=g) / 128.0
    mb = 1 + torch.randint(0, 128, (n,), generator=g) / 128.0
    gap = torch.randint(9, 31, (n,), generator=g).float()
    sa = torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0)
    sb = torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0)
    rows = torch.arange(n)
    big_first = torch.rand(n, generator=g) < 0.5
    x[rows, 2 * k + (~big_first).long()] = sa * ma * 4.0
    x[rows, 2 * k + big_first.long()] = sb * mb * 4.0 * torch.exp2(-gap)
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("d", [64, 128])
def test_encode_inexact_first_stage_bit_exact(dev, bits, d):
    x = wide_pair_rows(4096, 23, d)
    want_c, want_s = O.encode(bf16_bits(x), "bf16", bits, O.diag(42, d))
    codes, scale = PolarQuant(bits).encode(x.to(dev))
    np.testing.assert_array_equal(scale.cpu().numpy(), want_s)
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)


@pytest.mark.parametrize("bits,d,n", [(4, 128, 3001), (8, 128, 3001), (4, 64, 3001), (8, 64, 3001),
                                      (8, 128, 200003), (4, 64, 400003), (8, 64, 400003)])
def test_specialised_and_generic_encode_agree(dev, bits, d, n):
    # the production-shape kernels (4-bit D=128; 8-bit D=128 and 4/8-bit D=64 with the fp64
    # quantiser factor and the exact fallback for undecided waves) against the generic kernel and the
    # oracle; n not a multiple of a wave's vectors, the large n over thousands of waves (some of which
    # take the fallback)
    import aetherkv._lib as L

    x = normal_with_outliers((n, d), 5 + d + bits, trailing_dims=1).to(dev)
    pq = PolarQuant(bits)
    prev = L.lib().aekv_set_generic_kernels(1)
    try:
        cg, sg = pq.encode(x)
    finally:
        L.lib().aekv_set_generic_kernels(prev)
    cs, ss = pq.encode(x)
    assert torch.equal(cg, cs) and torch.equal(sg, ss)
    want_c, want_s = O.encode(bf16_bits(x), "bf16", bits, O.diag(42, d))
    np.testing.assert_array_equal(cs.cpu().numpy(), want_c)
    np.testing.assert_array_equal(ss.cpu().numpy(), want_s)


@pytest.mark.parametrize("n", [1, 15, 16, 4097, 262147])
def test_specialised_and_generic_decode_agree(dev, n):
    """4-bit D=128 bf16 decode: the quad-layout kernel against the generic one and the oracle,
    including scales of 2^124 and above (the kernel's exact-product fallback) and tiny scales.
    262147 vectors take the several-passes-per-wave launch (65537 passes, the last one partial)."""
    import aetherkv._lib as L

    rng = np.random.default_rng(n)
    codes = rng.integers(0, 256, (n, 64)).astype(np.uint8)
    scale = (rng.random((n, 1)) * 0.5 + 1e-3).astype(np.float32)
    scale[::7] = np.float32(3e37)   # above 2^124: the fallback path; one small code keeps the row finite
    codes[::7] = 0
    codes[::7, 5] = 0x3D
    scale[3::11] = np.float32(1.5e-38)
    scale[5::13] = np.float32(0.0)
    pq = PolarQuant(4)
    c, s = torch.from_numpy(codes).to(dev), torch.from_numpy(scale).to(dev)
    prev = L.lib().aekv_set_generic_kernels(1)
    try:
        gen = pq.decode(c, s)
    finally:
        L.lib().aekv_set_generic_kernels(prev)
    spec = pq.decode(c, s)
    assert torch.equal(bf16_bits_t(spec), bf16_bits_t(gen))
    np.testing.assert_array_equal(bf16_bits(spec), O.decode(codes, scale, 4, O.diag(42, 128), "bf16"))


def bf16_bits_t(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16)


def test_empty_and_misaligned_inputs(dev):
    pq = PolarQuant(4)
    c, s = pq.encode(torch.empty(0, 128, dtype=torch.bfloat16, device=dev))
    assert c.shape == (0, 64) and s.shape == (0, 1)
    assert pq.decode(c, s).shape == (0, 128)
    base = torch.randn(1 + 33 * 128, dtype=torch.bfloat16, device=dev)
    x = base[1:].view(33, 128)  # data pointer offset by 2 bytes
    c1, s1 = pq.encode(x)
    c2, s2 = pq.encode(x.clone())
    assert torch.equal(c1, c2) and torch.equal(s1, s2)


def test_encode_accepts_any_leading_shape(dev):
    x = torch.randn(2, 3, 5, 64, dtype=torch.bfloat16, device=dev)
    pq = PolarQuant(8)
    c, s = pq.encode(x)
    assert c.shape == (2, 3, 5, 64) and s.shape == (2, 3, 5, 1)
    c2, s2 = pq.encode(x.view(-1, 64))
    assert torch.equal(c.view(-1, 64), c2) and torch.equal(s.view(-1, 1), s2)
