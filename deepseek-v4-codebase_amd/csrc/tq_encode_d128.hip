// Fast TurboQuant 4-bit encode for the production shape: D = 128, bf16 input (gfx950).
//
// Same result, bit for bit, as tq_forward_kernel<BF16, 128, ENC4> and as
// aether_2b/turbo_quant.py:127-166 (rot = _wht(x*diag); m = max(max|rot|, 1e-8); scale = m/7;
// q = clamp(rne(rot/m*7)); nibble pack), with about half the VALU work:
//
// * Layout.  A wave handles 16 vectors; lane l = 16*g + v holds elements [32g, 32g+32) of vector
//   v (four 16-byte loads).  Butterfly stages h = 1..16 run in registers.  Stage h = 32 pairs lane
//   rows g0 = 0/1 and stage h = 64 pairs lane halves g1 = 0/1: one v_permlane16_swap /
//   v_permlane32_swap exchanges two registers so that every lane ends up holding (lower, upper)
//   of one pair and applies the same add/sub.  After both swaps lane (g1, g0) holds elements
//   e = 64*R4 + 32*g1 + 16*g0 + (R & 15) in register R, so its codes are two runs of 8 bytes.
// * x * diag and the first butterfly stage: per packed bf16 word, lo = w << 16, hi*diag = the
//   high half with its sign flipped by diag (one bitwise op), and a + b / a - b =
//   fma(lo, diag_lo, +-hi*diag) — an exact product and one rounding, i.e. the reference's fp32
//   add/sub.  (v_dot2_f32_bf16 computes the same sum but does not round it like an fp32 add when
//   the two halves are more than 2^16 apart, so it is not used.)
// * Scale folding.  max|rot| = RN(c * max|raw|) because rounding is monotonic (raw = butterfly
//   output before the * c, c = fp32(128^-0.5)), so the per-element work uses the exact product
//   P = raw * K with K = RN(RN(7c) * rcp(m)) (v_rcp_f32, relative error <= 2^-23) instead of
//   RN(RN(RN(raw*c)/m)*7).  |P/T - 1| <= 4 * 2^-24 and |t_exact/T - 1| <= 3 * 2^-24 for
//   T = raw*7c/m, |T| <= 7, so |P - t_exact| <= 49 * 2^-24 < 2.95e-6, and
//   rne(P) = rne(t_exact) unless P lies within that distance of a half-integer.  The kernel checks
//   max |P - rne(P)| over the wave and, if any element is within kDelta = 5e-6 of a tie, redoes
//   the wave's elements with the reference's exact operation sequence (~1e-5 per element).
// * rne(P) and the nibble come from one FMA with the magic constant M8 = 1.5 * 2^23 + 8:
//   RN(raw*K + M8) = M8 + rne(P), whose low byte is rne(P) + 8 (offset binary); a nibble pair is
//   one shift-or and one XOR with 0x88888888 per dword restores two's complement.
#include <atomic>
#include <cstdlib>
#include <cstring>

#include "tq_device.h"

namespace aekv {
namespace {

constexpr int kThreads = 256;
constexpr float kMagic8 = 12582920.0f;  // 1.5 * 2^23 + 8: RN(t + kMagic8) = kMagic8 + rne(t), ulp 1
constexpr float kDelta = 5e-6f;

__device__ __forceinline__ void swap16(float& a, float& b) {
  auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), false,
                                            false);
  a = __builtin_bit_cast(float, static_cast<uint32_t>(r[0]));
  b = __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

__device__ __forceinline__ void swap32(float& a, float& b) {
  auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), false,
                                            false);
  a = __builtin_bit_cast(float, static_cast<uint32_t>(r[0]));
  b = __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

// ue, uo: bit patterns of M8 + n (n in [-7, 7]), whose low byte is n + 8 in [1, 15].
// Returns a word whose low byte is (n_odd + 8) << 4 | (n_even + 8); bits 8.. are garbage.
__device__ __forceinline__ uint32_t nib_pair(uint32_t ue, uint32_t uo) { return (uo << 4) | ue; }

// Low bytes of four nib_pair words -> one dword of two's-complement nibbles (xor 8 per nibble
// turns the offset-binary n + 8 into n & 15).
__device__ __forceinline__ uint32_t pack4(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // [b0.0, b1.0, 0, 0]
  const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x04000c0cu);  // [0, 0, b2.0, b3.0]
  return (lo | hi) ^ 0x88888888u;
}

// max(acc, |x|, |y|) as one v_max3_f32 with abs source modifiers.
__device__ __forceinline__ float max3_abs(float acc, float x, float y) {
  float r;
  asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(acc), "v"(x), "v"(y));
  return r;
}

__global__ __launch_bounds__(kThreads) void tq_encode4_d128_bf16_kernel(const uint32_t* __restrict__ x,
                                                                        int64_t n_vec,
                                                                        const float* __restrict__ diag, float c,
                                                                        float c7, uint8_t* __restrict__ codes,
                                                                        float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int v = lane & 15, g = lane >> 4, g0 = g & 1, g1 = g >> 1;

  // diag of the packed words this lane loads: diag[32g + 2k] as +-1, diag[32g + 2k + 1] as a sign mask
  float dlo[16];
  uint32_t shi[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    dlo[k] = diag[32 * g + 2 * k];
    shi[k] = diag[32 * g + 2 * k + 1] < 0.0f ? 0x80000000u : 0u;
  }

  const int64_t n_groups = (n_vec + 15) >> 4;
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 6;
  const int64_t n_waves = (static_cast<int64_t>(gridDim.x) * kThreads) >> 6;
  for (int64_t grp = wave; grp < n_groups; grp += n_waves) {
    const int64_t vec = grp * 16 + v;
    const bool ok = vec < n_vec;
    // lanes past the end re-read the last vector (never stored) so every lane runs the same code
    const uint4* p = reinterpret_cast<const uint4*>(x + (ok ? vec : n_vec - 1) * 64 + g * 16);
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 t = p[i];
      w[4 * i] = t.x;
      w[4 * i + 1] = t.y;
      w[4 * i + 2] = t.z;
      w[4 * i + 3] = t.w;
    }
    float a[32];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      // stage h = 1 on x * diag: lo + hi, lo - hi
      const float lo = __builtin_bit_cast(float, w[k] << 16);
      const float hs = __builtin_bit_cast(float, (w[k] & 0xFFFF0000u) ^ shi[k]);
      a[2 * k] = fmaf(lo, dlo[k], hs);
      a[2 * k + 1] = fmaf(lo, dlo[k], -hs);
    }
    // stages h = 2, 4, 8, 16 in registers
#pragma unroll
    for (int h = 2; h < 32; h <<= 1) {
#pragma unroll
      for (int blk = 0; blk < 32; blk += 2 * h) {
#pragma unroll
        for (int i = 0; i < h; ++i) {
          const float p = a[blk + i], q = a[blk + h + i];
          a[blk + i] = p + q;
          a[blk + h + i] = p - q;
        }
      }
    }
    // stage h = 32 (element bit 5 = lane bit 4): afterwards reg r + 16s holds element 32s + 16g0 + r
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      swap16(a[r], a[r + 16]);
      const float p = a[r], q = a[r + 16];
      a[r] = p + q;
      a[r + 16] = p - q;
    }
    // stage h = 64 (element bit 6 = lane bit 5): afterwards reg R holds 64*R4 + 32g1 + 16g0 + (R&15)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      swap32(a[r], a[r + 16]);
      const float p = a[r], q = a[r + 16];
      a[r] = p + q;
      a[r + 16] = p - q;
    }

    // m = max(RN(c * max|raw|), 1e-8) over the 4 lanes of the vector
    float mr = 0.0f;
#pragma unroll
    for (int r = 0; r < 32; r += 2) mr = max3_abs(mr, a[r], a[r + 1]);
    mr = fmaxf(mr, xor_lane<16>(mr));
    mr = fmaxf(mr, xor_lane<32>(mr));
    const float m = fmaxf(mr * c, 1e-8f);
    const float K = c7 * __builtin_amdgcn_rcpf(m);  // v_rcp_f32: 1 ulp; only feeds the checked fast path

    // fast path: u = RN(a*K + M8) = M8 + rne(a*K) (exact product, one rounding), d = a*K - n
    uint32_t o[4];
    float md = 0.0f;
#pragma unroll
    for (int dw = 0; dw < 4; ++dw) {
      uint32_t b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x0 = a[8 * dw + 2 * j], x1 = a[8 * dw + 2 * j + 1];
        const float u0 = fmaf(x0, K, kMagic8), u1 = fmaf(x1, K, kMagic8);
        md = max3_abs(md, fmaf(x0, K, kMagic8 - u0), fmaf(x1, K, kMagic8 - u1));
        b[j] = nib_pair(__builtin_bit_cast(uint32_t, u0), __builtin_bit_cast(uint32_t, u1));
      }
      o[dw] = pack4(b[0], b[1], b[2], b[3]);
    }
    if (__builtin_amdgcn_ballot_w64(md > 0.5f - kDelta) != 0) {
      // a tie is within reach of the fast path's error: the reference's exact sequence
#pragma unroll
      for (int dw = 0; dw < 4; ++dw) {
        uint32_t b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float t0 = (a[8 * dw + 2 * j] * c) / m, t1 = (a[8 * dw + 2 * j + 1] * c) / m;
          t0 = t0 * 7.0f;
          t1 = t1 * 7.0f;
          b[j] = nib_pair(__builtin_bit_cast(uint32_t, rintf(t0) + kMagic8),
                          __builtin_bit_cast(uint32_t, rintf(t1) + kMagic8));
        }
        o[dw] = pack4(b[0], b[1], b[2], b[3]);
      }
    }
    if (ok) {
      if (g == 0) scale[vec] = m / 7.0f;
      uint8_t* cp = codes + vec * 64 + 8 * (g0 + 2 * g1);
      *reinterpret_cast<uint2*>(cp) = make_uint2(o[0], o[1]);       // elements 16g' .. 16g'+15
      *reinterpret_cast<uint2*>(cp + 32) = make_uint2(o[2], o[3]);  // elements 64 + 16g' ..
    }
  }
}

}  // namespace

namespace {
std::atomic<int> g_generic_only{-1};  // -1: not yet read from the environment
}

bool use_specialised_codec() {
  int v = g_generic_only.load(std::memory_order_relaxed);
  if (v < 0) {
    const char* e = std::getenv("AETHERKV_CODEC");
    v = (e && std::strcmp(e, "generic") == 0) ? 1 : 0;
    g_generic_only.store(v, std::memory_order_relaxed);
  }
  return v == 0;
}

}  // namespace aekv

extern "C" int aekv_set_generic_kernels(int generic_only) {
  (void)aekv::use_specialised_codec();
  return aekv::g_generic_only.exchange(generic_only ? 1 : 0);
}

namespace aekv {

// Launches the specialised kernel; returns false when the shape is not the specialised one.
bool launch_encode4_d128_bf16(const void* x, int64_t n_vec, const float* diag, float c, void* codes, float* scale,
                              hipStream_t st) {
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(codes) & 7)) return false;
  const int64_t n_groups = (n_vec + 15) / 16;
  int64_t blocks = ceil_div(n_groups, kThreads / 64);
  if (blocks > 8192) blocks = 8192;  // grid-stride beyond 32768 waves
  const float c7 = c * 7.0f;
  hipLaunchKernelGGL(tq_encode4_d128_bf16_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, st,
                     static_cast<const uint32_t*>(x), n_vec, diag, c, c7, static_cast<uint8_t*>(codes), scale);
  return true;
}

}  // namespace aekv
