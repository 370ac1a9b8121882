// TurboQuant ("PolarQuant") codec for gfx950: normalised Walsh-Hadamard transform, absmax
// 8/4-bit quantisation with nibble packing, and the inverse.
//
// Reference: aether_2b/turbo_quant.py:49-76 (_wht), :127-166 (encode), :168-211 (decode).
// Bit-exact with the reference: every fp32 operation of the reference is performed once, in the
// same order, with the same rounding (the library is built with -ffp-contract=off; the only FMAs
// are the explicit fmaf(a, +-1, b) below, whose product is exact).
//
// Layout: a vector of D elements is spread over LPV = D/EPL lanes, EPL = min(D, 8) consecutive
// elements per lane, so one lane's load is one 16-byte access for bf16 and a wave reads 64*16
// contiguous bytes.  Butterfly stages h = 1..EPL/2 run inside the lane; stages h = EPL..D/2 pair
// lane l with lane l ^ (h/EPL) (DPP for 1/2, ds_swizzle for 4/8/16, ds_bpermute for 32).  The
// butterfly result for the lane holding the upper element is partner - mine, for the lower one
// mine + partner; both are one fmaf(mine, +-1, partner).
#include "tq_device.h"

namespace aekv {
namespace {

constexpr int kThreads = 256;
enum { kModeWht = 0, kModeEnc4 = 4, kModeEnc8 = 8 };

// Forward kernel: WHT (fp32 out), or encode to 8/4-bit codes + fp32 scale.
template <int DT, int D, int MODE>
__global__ __launch_bounds__(kThreads) void tq_forward_kernel(const void* __restrict__ x, int64_t n_vec,
                                                              const float* __restrict__ diag, float c,
                                                              void* __restrict__ out,
                                                              float* __restrict__ out_scale) {
  constexpr int EPL = D < 8 ? D : 8;
  constexpr int LPV = D / EPL;
  constexpr int VPW = 64 / LPV;
  const int lane = threadIdx.x & 63;
  const int sub = lane % LPV;
  const int slot = lane / LPV;

  float dg[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) dg[e] = MODE == kModeWht ? 1.0f : diag[sub * EPL + e];

  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 6;
  const int64_t n_waves = (static_cast<int64_t>(gridDim.x) * kThreads) >> 6;
  for (int64_t base = wave * VPW; base < n_vec; base += n_waves * VPW) {
    const int64_t v = base + slot;
    const bool ok = v < n_vec;
    float a[EPL];
    load_elems<DT, EPL>(x, v * D + sub * EPL, ok, a);
    if constexpr (MODE == kModeWht) {
      wht_butterflies<D, EPL, true>(a, sub);
      if (ok) {
        float* o = static_cast<float*>(out) + v * D + sub * EPL;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[e] = a[e] * c;  // * fp32(d ** -0.5)
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPL; ++e) a[e] = a[e] * dg[e];  // x.float() * diag (exact sign flip)
      constexpr int BITS = MODE == kModeEnc8 ? 8 : 4;
      constexpr int NB = BITS == 8 ? EPL : EPL / 2;
      float m;
      const Bytes<NB> w = encode_lane<BITS, D, true>(a, sub, c, &m);
      if (ok) {
        if (sub == 0) out_scale[v] = m / (BITS == 8 ? 127.0f : 7.0f);
        *reinterpret_cast<Bytes<NB>*>(static_cast<uint8_t*>(out) + v * (BITS == 8 ? D : D / 2) + sub * NB) = w;
      }
    }
  }
}

// Decode kernel: codes * scale -> WHT -> * diag -> out dtype.
template <int BITS, int D, int ODT>
__global__ __launch_bounds__(kThreads) void tq_decode_kernel(const void* __restrict__ codes,
                                                             const float* __restrict__ scale, int64_t n_vec,
                                                             const float* __restrict__ diag, float c,
                                                             void* __restrict__ out) {
  constexpr int EPL = D < 8 ? D : 8;
  constexpr int LPV = D / EPL;
  constexpr int VPW = 64 / LPV;
  const int lane = threadIdx.x & 63;
  const int sub = lane % LPV;
  const int slot = lane / LPV;

  float dg[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) dg[e] = diag[sub * EPL + e];

  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 6;
  const int64_t n_waves = (static_cast<int64_t>(gridDim.x) * kThreads) >> 6;
  for (int64_t base = wave * VPW; base < n_vec; base += n_waves * VPW) {
    const int64_t v = base + slot;
    const bool ok = v < n_vec;
    float a[EPL];
    // inactive lanes decode row 0 so every lane joins the cross-lane butterflies
    const int64_t vr = ok ? v : 0;
    decode_lane<BITS, D, true>(static_cast<const uint8_t*>(codes) + vr * (BITS == 8 ? D : D / 2), scale[vr], sub, dg, c, a);
    if (ok) {
      uint8_t* o = static_cast<uint8_t*>(out) + (v * D + sub * EPL) * (ODT == AEKV_F32 ? 4 : 2);
      if constexpr (ODT == AEKV_F32) {
        Bytes<EPL * 4> w;
        __builtin_memcpy(w.b, a, EPL * 4);
        if constexpr (EPL * 4 <= 16) {
          *reinterpret_cast<Bytes<EPL * 4>*>(o) = w;
        } else {
          reinterpret_cast<Bytes<16>*>(o)[0] = *reinterpret_cast<Bytes<16>*>(w.b);
          reinterpret_cast<Bytes<16>*>(o)[1] = *reinterpret_cast<Bytes<16>*>(w.b + 16);
        }
      } else if constexpr (ODT == AEKV_BF16) {
        if constexpr (EPL >= 2) {
          uint32_t wv[EPL / 2];
#pragma unroll
          for (int i = 0; i < EPL / 2; ++i) wv[i] = pack_bf16x2(a[2 * i], a[2 * i + 1]);
          Bytes<EPL * 2> w;
          __builtin_memcpy(w.b, wv, EPL * 2);
          *reinterpret_cast<Bytes<EPL * 2>*>(o) = w;
        } else {
          *reinterpret_cast<uint16_t*>(o) = static_cast<uint16_t>(pack_bf16x2(a[0], 0.0f) & 0xffffu);
        }
      } else {
        Bytes<EPL * 2> w;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const uint16_t h = static_cast<uint16_t>(f32_to_f16_bits(a[e]));
          __builtin_memcpy(w.b + 2 * e, &h, 2);
        }
        *reinterpret_cast<Bytes<EPL * 2>*>(o) = w;
      }
    }
  }
}

int64_t grid_for(int64_t n_vec, int d) {
  const int epl = d < 8 ? d : 8;
  const int vpb = (64 / (d / epl)) * (kThreads / 64);  // vectors per block per iteration
  int64_t g = ceil_div(n_vec, vpb);
  if (g > 65536) g = 65536;
  return g < 1 ? 1 : g;
}

typedef void (*fwd_fn)(const void*, int64_t, const float*, float, void*, float*);
typedef void (*dec_fn)(const void*, const float*, int64_t, const float*, float, void*);

template <int DT, int MODE>
fwd_fn pick_fwd(int d) {
  switch (d) {
    case 1: return MODE == kModeEnc4 ? nullptr : tq_forward_kernel<DT, 1, MODE>;
    case 2: return tq_forward_kernel<DT, 2, MODE>;
    case 4: return tq_forward_kernel<DT, 4, MODE>;
    case 8: return tq_forward_kernel<DT, 8, MODE>;
    case 16: return tq_forward_kernel<DT, 16, MODE>;
    case 32: return tq_forward_kernel<DT, 32, MODE>;
    case 64: return tq_forward_kernel<DT, 64, MODE>;
    case 128: return tq_forward_kernel<DT, 128, MODE>;
    case 256: return tq_forward_kernel<DT, 256, MODE>;
    case 512: return tq_forward_kernel<DT, 512, MODE>;
    default: return nullptr;
  }
}

template <int MODE>
fwd_fn pick_fwd_dt(int dt, int d) {
  if (dt == AEKV_F32) return pick_fwd<AEKV_F32, MODE>(d);
  if (dt == AEKV_F16) return pick_fwd<AEKV_F16, MODE>(d);
  return pick_fwd<AEKV_BF16, MODE>(d);
}

template <int BITS, int ODT>
dec_fn pick_dec(int d) {
  switch (d) {
    case 1: return BITS == 4 ? nullptr : tq_decode_kernel<BITS, 1, ODT>;
    case 2: return tq_decode_kernel<BITS, 2, ODT>;
    case 4: return tq_decode_kernel<BITS, 4, ODT>;
    case 8: return tq_decode_kernel<BITS, 8, ODT>;
    case 16: return tq_decode_kernel<BITS, 16, ODT>;
    case 32: return tq_decode_kernel<BITS, 32, ODT>;
    case 64: return tq_decode_kernel<BITS, 64, ODT>;
    case 128: return tq_decode_kernel<BITS, 128, ODT>;
    case 256: return tq_decode_kernel<BITS, 256, ODT>;
    case 512: return tq_decode_kernel<BITS, 512, ODT>;
    default: return nullptr;
  }
}

template <int BITS>
dec_fn pick_dec_dt(int odt, int d) {
  if (odt == AEKV_F32) return pick_dec<BITS, AEKV_F32>(d);
  if (odt == AEKV_F16) return pick_dec<BITS, AEKV_F16>(d);
  return pick_dec<BITS, AEKV_BF16>(d);
}

int check_vec_dim(int32_t d) {
  if (!is_pow2(d)) return fail(AEKV_ERR_VALUE, "WHT requires last dim to be a power of 2, got %d", d);
  if (d > 512) return fail(AEKV_ERR_UNSUPPORTED, "vector length %d exceeds the supported maximum 512", d);
  return AEKV_OK;
}

}  // namespace
}  // namespace aekv

using namespace aekv;

extern "C" int aekv_wht(const void* x, int32_t x_dtype, int64_t n_vec, int32_t d, float* out, void* stream) {
  if (int rc = check_vec_dim(d)) return rc;
  if (!is_float_dtype(x_dtype)) return fail(AEKV_ERR_DTYPE, "aekv_wht: x_dtype %d is not f32/f16/bf16", x_dtype);
  if (n_vec < 0) return fail(AEKV_ERR_SHAPE, "aekv_wht: n_vec %lld < 0", (long long)n_vec);
  if (n_vec == 0) return AEKV_OK;
  if (!x || !out) return fail(AEKV_ERR_VALUE, "aekv_wht: null pointer");
  const int epl = d < 8 ? d : 8;
  if (!is_aligned(x, epl * dtype_size(x_dtype) > 16 ? 16 : epl * dtype_size(x_dtype)) || !is_aligned(out, 4))
    return fail(AEKV_ERR_ALIGN, "aekv_wht: misaligned pointer");
  fwd_fn fn = pick_fwd_dt<kModeWht>(x_dtype, d);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(grid_for(n_vec, d))), dim3(kThreads), 0, as_stream(stream), x,
                     n_vec, nullptr, wht_scale(d), static_cast<void*>(out), nullptr);
  return check_launch("aekv_wht");
}

extern "C" int aekv_tq_encode(const void* x, int32_t x_dtype, int64_t n_vec, int32_t d, int32_t bits,
                              const float* diag, void* codes, float* scale, void* stream) {
  if (bits != 4 && bits != 8) return fail(AEKV_ERR_VALUE, "bits must be 4 or 8, got %d", bits);
  if (int rc = check_vec_dim(d)) return rc;
  if (bits == 4 && d < 2) return fail(AEKV_ERR_VALUE, "4-bit packing needs an even last dim, got %d", d);
  if (!is_float_dtype(x_dtype)) return fail(AEKV_ERR_DTYPE, "aekv_tq_encode: x_dtype %d is not f32/f16/bf16", x_dtype);
  if (n_vec < 0) return fail(AEKV_ERR_SHAPE, "aekv_tq_encode: n_vec %lld < 0", (long long)n_vec);
  if (n_vec == 0) return AEKV_OK;
  if (!x || !diag || !codes || !scale) return fail(AEKV_ERR_VALUE, "aekv_tq_encode: null pointer");
  const int epl = d < 8 ? d : 8;
  const size_t in_al = epl * dtype_size(x_dtype) > 16 ? 16 : epl * dtype_size(x_dtype);
  const size_t out_al = bits == 8 ? epl : epl / 2;
  if (!is_aligned(x, in_al) || !is_aligned(codes, out_al) || !is_aligned(scale, 4) || !is_aligned(diag, 4))
    return fail(AEKV_ERR_ALIGN, "aekv_tq_encode: misaligned pointer (x needs %zu, codes %zu bytes)", in_al, out_al);
  if (bits == 4 && d == 128 && x_dtype == AEKV_BF16 && use_specialised_codec() &&
      launch_encode4_d128_bf16(x, n_vec, diag, wht_scale(d), codes, scale, as_stream(stream)))
    return check_launch("aekv_tq_encode");
  if (x_dtype == AEKV_BF16 && use_specialised_codec() &&
      launch_encode_fast_bf16(x, n_vec, bits, d, diag, wht_scale(d), codes, scale, as_stream(stream)))
    return check_launch("aekv_tq_encode");
  fwd_fn fn = bits == 8 ? pick_fwd_dt<kModeEnc8>(x_dtype, d) : pick_fwd_dt<kModeEnc4>(x_dtype, d);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(grid_for(n_vec, d))), dim3(kThreads), 0, as_stream(stream), x,
                     n_vec, diag, wht_scale(d), codes, scale);
  return check_launch("aekv_tq_encode");
}

extern "C" int aekv_tq_decode(const void* codes, const float* scale, int64_t n_vec, int32_t d, int32_t bits,
                              const float* diag, void* out, int32_t out_dtype, void* stream) {
  if (bits != 4 && bits != 8) return fail(AEKV_ERR_VALUE, "bits must be 4 or 8, got %d", bits);
  if (int rc = check_vec_dim(d)) return rc;
  if (bits == 4 && d < 2) return fail(AEKV_ERR_VALUE, "4-bit packing needs an even last dim, got %d", d);
  if (!is_float_dtype(out_dtype)) return fail(AEKV_ERR_DTYPE, "aekv_tq_decode: out_dtype %d is not f32/f16/bf16", out_dtype);
  if (n_vec < 0) return fail(AEKV_ERR_SHAPE, "aekv_tq_decode: n_vec %lld < 0", (long long)n_vec);
  if (n_vec == 0) return AEKV_OK;
  if (!codes || !scale || !diag || !out) return fail(AEKV_ERR_VALUE, "aekv_tq_decode: null pointer");
  const int epl = d < 8 ? d : 8;
  const size_t in_al = bits == 8 ? epl : epl / 2;
  const size_t out_al = epl * dtype_size(out_dtype) > 16 ? 16 : epl * dtype_size(out_dtype);
  if (!is_aligned(codes, in_al) || !is_aligned(out, out_al) || !is_aligned(scale, 4) || !is_aligned(diag, 4))
    return fail(AEKV_ERR_ALIGN, "aekv_tq_decode: misaligned pointer (codes needs %zu, out %zu bytes)", in_al, out_al);
  if (bits == 4 && d == 128 && out_dtype == AEKV_BF16 && use_specialised_codec() &&
      launch_decode4_d128_bf16(codes, scale, n_vec, diag, wht_scale(d), out, as_stream(stream)))
    return check_launch("aekv_tq_decode");
  dec_fn fn = bits == 8 ? pick_dec_dt<8>(out_dtype, d) : pick_dec_dt<4>(out_dtype, d);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(grid_for(n_vec, d))), dim3(kThreads), 0, as_stream(stream),
                     codes, scale, n_vec, diag, wht_scale(d), out);
  return check_launch("aekv_tq_decode");
}
