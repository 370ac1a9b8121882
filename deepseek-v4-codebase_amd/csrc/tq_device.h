// Device-side building blocks of the TurboQuant codec, shared by the codec kernels and by the
// attention kernels that dequantise KV codes on load.
//
// Layout: a D-element vector is spread over LPV = D/EPL lanes with EPL = min(D, 8) consecutive
// elements per lane.  Butterfly stages h < EPL run inside a lane; stage h >= EPL pairs lane l with
// lane l ^ (h/EPL).  Every fp32 operation of aether_2b/turbo_quant.py:49-211 is performed once, in
// the reference's order, so results are bit-exact (the library is built with -ffp-contract=off).
#pragma once

#include "aekv_common.h"

namespace aekv {

template <int N>
struct alignas(N) Bytes {
  uint8_t b[N];
};

// Load EPL elements of type dtype (F32/F16/BF16) starting at element offset `off`.
template <int DT, int EPL>
__device__ __forceinline__ void load_elems(const void* base, int64_t off, bool ok, float (&a)[EPL]) {
  constexpr int ES = DT == AEKV_F32 ? 4 : 2;
  constexpr int NB = ES * EPL;
  if (!ok) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) a[e] = 0.0f;
    return;
  }
  const uint8_t* p = static_cast<const uint8_t*>(base) + off * ES;
  if constexpr (NB <= 16) {
    Bytes<NB> raw = *reinterpret_cast<const Bytes<NB>*>(p);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      if constexpr (DT == AEKV_F32) {
        uint32_t u;
        __builtin_memcpy(&u, raw.b + 4 * e, 4);
        a[e] = __builtin_bit_cast(float, u);
      } else {
        uint16_t u;
        __builtin_memcpy(&u, raw.b + 2 * e, 2);
        a[e] = DT == AEKV_BF16 ? bf16_to_f32(u) : f16_to_f32(u);
      }
    }
  } else {  // fp32, EPL == 8: two 16-byte loads (as vectors: byte arrays copied out of end up in scratch)
    const float4 r0 = reinterpret_cast<const float4*>(p)[0];
    const float4 r1 = reinterpret_cast<const float4*>(p)[1];
    a[0] = r0.x;
    a[1] = r0.y;
    a[2] = r0.z;
    a[3] = r0.w;
    a[4] = r1.x;
    a[5] = r1.y;
    a[6] = r1.z;
    a[7] = r1.w;
  }
}

template <int HL, int EPL, bool LDS_PIPE = false>
__device__ __forceinline__ void cross_stage(float (&a)[EPL], int sub) {
  const float s = (sub & HL) ? -1.0f : 1.0f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float p = xor_lane<HL, LDS_PIPE>(a[e]);
    a[e] = fmaf(a[e], s, p);  // lower lane: a + p ; upper lane: p - a   (product exact)
  }
}

// Butterfly stages of a D-point transform spread over LPV lanes x EPL elements.  LDS_PIPE selects
// the lane-exchange path (see xor_lane).
template <int D, int EPL, bool LDS_PIPE = false>
__device__ __forceinline__ void wht_butterflies(float (&a)[EPL], int sub) {
  constexpr int LPV = D / EPL;
#pragma unroll
  for (int h = 1; h < EPL; h <<= 1) {
#pragma unroll
    for (int blk = 0; blk < EPL; blk += 2 * h) {
#pragma unroll
      for (int i = 0; i < h; ++i) {
        const float x = a[blk + i], y = a[blk + h + i];
        a[blk + i] = x + y;
        a[blk + h + i] = x - y;
      }
    }
  }
  if constexpr (LPV > 1) cross_stage<1, EPL, LDS_PIPE>(a, sub);
  if constexpr (LPV > 2) cross_stage<2, EPL, LDS_PIPE>(a, sub);
  if constexpr (LPV > 4) cross_stage<4, EPL, LDS_PIPE>(a, sub);
  if constexpr (LPV > 8) cross_stage<8, EPL, LDS_PIPE>(a, sub);
  if constexpr (LPV > 16) cross_stage<16, EPL, LDS_PIPE>(a, sub);
  if constexpr (LPV > 32) cross_stage<32, EPL, LDS_PIPE>(a, sub);
}

template <int D, int EPL, bool LDS_PIPE = false>
__device__ __forceinline__ float group_absmax(const float (&a)[EPL]) {
  constexpr int LPV = D / EPL;
  float m = 0.0f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) m = fmaxf(m, fabsf(a[e]));
  if constexpr (LPV > 1) m = fmaxf(m, xor_lane<1, LDS_PIPE>(m));
  if constexpr (LPV > 2) m = fmaxf(m, xor_lane<2, LDS_PIPE>(m));
  if constexpr (LPV > 4) m = fmaxf(m, xor_lane<4, LDS_PIPE>(m));
  if constexpr (LPV > 8) m = fmaxf(m, xor_lane<8, LDS_PIPE>(m));
  if constexpr (LPV > 16) m = fmaxf(m, xor_lane<16, LDS_PIPE>(m));
  if constexpr (LPV > 32) m = fmaxf(m, xor_lane<32, LDS_PIPE>(m));
  return m;
}


// Encode of the EPL elements of one vector held by this lane, from x * diag (turbo_quant.py:
// 127-166): WHT, * c, m = max(max|rot|, 1e-8) over the vector's lanes, q = clamp(rne(rot/m * Q)),
// Q = 127 (8-bit) or 7 (4-bit).  Returns the lane's code bytes; *m_out = m (the scale is m / Q).
template <int BITS, int D, bool LDS_PIPE>
__device__ __forceinline__ Bytes<(BITS == 8 ? (D < 8 ? D : 8) : (D < 8 ? D : 8) / 2)> encode_lane(
    float (&a)[(D < 8 ? D : 8)], int sub, float c, float* m_out) {
  constexpr int EPL = D < 8 ? D : 8;
  constexpr float Q = BITS == 8 ? 127.0f : 7.0f;
  wht_butterflies<D, EPL, LDS_PIPE>(a, sub);
#pragma unroll
  for (int e = 0; e < EPL; ++e) a[e] = a[e] * c;  // * fp32(d ** -0.5)
  float m = group_absmax<D, EPL, LDS_PIPE>(a);
  m = fmaxf(m, 1e-8f);  // clamp_(min=1e-8)
  int q[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    float t = a[e] / m;  // correctly rounded division (-fhip-fp32-correctly-rounded-divide-sqrt)
    t = t * Q;
    t = rintf(t);  // round half to even
    t = fminf(fmaxf(t, -Q), Q);
    q[e] = static_cast<int>(t);
  }
  *m_out = m;
  Bytes<(BITS == 8 ? EPL : EPL / 2)> w;
  if constexpr (BITS == 8) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) w.b[e] = static_cast<uint8_t>(q[e] & 0xff);
  } else {
#pragma unroll
    for (int i = 0; i < EPL / 2; ++i) w.b[i] = static_cast<uint8_t>((q[2 * i] & 0x0f) | ((q[2 * i + 1] & 0x0f) << 4));
  }
  return w;
}

// Code bytes a lane holds for its EPL elements of one vector.
template <int BITS, int D>
struct LaneCodes {
  static constexpr int EPL = D < 8 ? D : 8;
  static constexpr int NB = BITS == 8 ? EPL : EPL / 2;  // code bytes per lane
  using type = Bytes<NB>;
};

// Dequantise the EPL elements of one vector held by this lane: codes * scale -> WHT -> * c -> * diag
// (turbo_quant.py:187-211), from the lane's code bytes (bytes sub*NB .. of the vector's row).
template <int BITS, int D, bool LDS_PIPE = false>
__device__ __forceinline__ void decode_lane_bytes(const typename LaneCodes<BITS, D>::type& w, float s, int sub,
                                                  const float (&dg)[(D < 8 ? D : 8)], float c,
                                                  float (&a)[(D < 8 ? D : 8)]) {
  constexpr int EPL = D < 8 ? D : 8;
  constexpr int NB = LaneCodes<BITS, D>::NB;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    if constexpr (BITS == 8) {
      a[i] = static_cast<float>(static_cast<int8_t>(w.b[i])) * s;
    } else {
      const int lo = (static_cast<int>(w.b[i] & 0x0f) ^ 8) - 8;  // sign-extend nibble
      const int hi = (static_cast<int>(w.b[i] >> 4) ^ 8) - 8;
      a[2 * i] = static_cast<float>(lo) * s;
      a[2 * i + 1] = static_cast<float>(hi) * s;
    }
  }
  wht_butterflies<D, EPL, LDS_PIPE>(a, sub);
#pragma unroll
  for (int e = 0; e < EPL; ++e) a[e] = (a[e] * c) * dg[e];
}

// The same, loading the lane's bytes from `row`, the vector's code row.
template <int BITS, int D, bool LDS_PIPE = false>
__device__ __forceinline__ void decode_lane(const uint8_t* __restrict__ row, float s, int sub,
                                            const float (&dg)[(D < 8 ? D : 8)], float c,
                                            float (&a)[(D < 8 ? D : 8)]) {
  using W = typename LaneCodes<BITS, D>::type;
  const W w = *reinterpret_cast<const W*>(row + sub * LaneCodes<BITS, D>::NB);
  decode_lane_bytes<BITS, D, LDS_PIPE>(w, s, sub, dg, c, a);
}

// Specialised production-shape kernels (tq_codec_d128.hip).  Each returns false (and launches
// nothing) when its alignment requirements are not met, so the caller falls back to the generic
// kernel.  AETHERKV_CODEC=generic in the environment forces the generic kernels (testing aid).
bool launch_encode4_d128_bf16(const void* x, int64_t n_vec, const float* diag, float c, void* codes, float* scale,
                              hipStream_t st);
bool launch_decode4_d128_bf16(const void* codes, const float* scale, int64_t n_vec, const float* diag, float c,
                              void* out, hipStream_t st);
// 8-bit D = 128 and 4- / 8-bit D = 64 encode, bf16 in.
bool launch_encode_fast_bf16(const void* x, int64_t n_vec, int bits, int d, const float* diag, float c, void* codes,
                             float* scale, hipStream_t st);

}  // namespace aekv
