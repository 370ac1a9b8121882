// RoPE then RMSNorm of head vectors in one pass: the attention step's query and window-entry
// preparation and its inverse RoPE on the output.
//
// Reference: aether_2b/serving.py:437-442 (_query: q_norm(apply_rope(q_up(latent), position))),
// :444-448 (_window_entry: kv_norm(apply_rope(window_kv(x), position))), :469-472
// (_post_attention: apply_rope(out, -position) before the output projection); apply_rope
// modeling.py:122-155, RMSNorm :32-41.  Torch runs these as separate bf16 ops; this kernel keeps
// their rounding points:
//   RoPE on the last rope_dim dims, pairs (2i, 2i+1) of that part, angle = fp32(sign * pos) * f_i,
//   cos/sin = bf16(cos/sin(angle)): even bf16(bf16(a cos) + bf16(-b sin)), odd
//   bf16(bf16(b cos) + bf16(a sin))
//   RMSNorm: r = 1 / sqrt(mean(x^2) + eps) in fp32, y = bf16((x * r) * w)
// Only the library cos/sin/sqrt and the order of the mean's sum can differ from torch's CPU
// kernels, i.e. an ulp of fp32 before a bf16 rounding.
//
// One wave per head vector; lane l holds dims [l * D/64, (l + 1) * D/64), so every RoPE pair is in
// one lane and the RMS is one wave sum.
#include "tq_device.h"

namespace aekv {
namespace {

struct RopeNormArgs {
  const uint16_t* x;      // [n_vec, D] bf16 (n_vec = rows * heads)
  const int64_t* pos;     // [rows]
  const float* inv_freq;  // [rope_dim / 2]
  const uint16_t* norm;   // [D] bf16 or null
  int64_t n_vec;
  int heads, rope_dim, sign;
  float eps;
  uint16_t* out;          // [n_vec, D] bf16
};

__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(pack_bf16x2(v, 0.0f) & 0xFFFFu); }

template <int D>
__global__ __launch_bounds__(256) void rope_rmsnorm_kernel(RopeNormArgs a) {
  constexpr int EPL = D / 64;
  const int lane = threadIdx.x & 63;
  const int64_t vec = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (vec >= a.n_vec) return;  // wave-uniform
  const int64_t row = vec / a.heads;
  const int d0 = lane * EPL;
  uint32_t w[EPL / 2];
  if constexpr (EPL == 2) {
    w[0] = *reinterpret_cast<const uint32_t*>(a.x + vec * D + d0);
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(a.x + vec * D + d0);
    w[0] = v.x;
    w[1] = v.y;
  }
  float x[EPL];
#pragma unroll
  for (int k = 0; k < EPL / 2; ++k) {
    x[2 * k] = __builtin_bit_cast(float, w[k] << 16);
    x[2 * k + 1] = __builtin_bit_cast(float, w[k] & 0xFFFF0000u);
  }
  if (a.rope_dim > 0) {
    const int r0 = D - a.rope_dim;
    const float p = static_cast<float>(static_cast<int64_t>(a.sign) * a.pos[row]);
#pragma unroll
    for (int e = 0; e < EPL; e += 2) {
      const int d = d0 + e;
      if (d >= r0) {
        const float ang = p * a.inv_freq[(d - r0) >> 1];
        const float cs = bf16r(cosf(ang)), sn = bf16r(sinf(ang));
        const float xa = x[e], xb = x[e + 1];
        x[e] = bf16r(bf16r(xa * cs) + bf16r(-xb * sn));
        x[e + 1] = bf16r(bf16r(xb * cs) + bf16r(xa * sn));
      }
    }
  }
  if (a.norm) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) ss += x[e] * x[e];
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(D) + a.eps);
#pragma unroll
    for (int e = 0; e < EPL; ++e) x[e] = bf16r((x[e] * r) * bf16_to_f32(a.norm[d0 + e]));
  }
  uint32_t o[EPL / 2];
#pragma unroll
  for (int k = 0; k < EPL / 2; ++k) o[k] = pack_bf16x2(x[2 * k], x[2 * k + 1]);
  if constexpr (EPL == 2) {
    *reinterpret_cast<uint32_t*>(a.out + vec * D + d0) = o[0];
  } else {
    *reinterpret_cast<uint2*>(a.out + vec * D + d0) = make_uint2(o[0], o[1]);
  }
}

}  // namespace
}  // namespace aekv

using namespace aekv;

extern "C" int aekv_rope_rmsnorm(const void* x, int64_t rows, int32_t heads, int32_t d, const int64_t* positions,
                                 int32_t pos_sign, const float* inv_freq, int32_t rope_dim, const void* norm_weight,
                                 float eps, void* out, void* stream) {
  const char* who = "aekv_rope_rmsnorm";
  if (d != 128 && d != 256) return fail(AEKV_ERR_UNSUPPORTED, "%s: head dim %d (128 or 256 supported)", who, d);
  if (rows < 0 || heads < 1) return fail(AEKV_ERR_SHAPE, "%s: rows=%lld heads=%d", who, (long long)rows, heads);
  if (rope_dim < 0 || rope_dim > d || (rope_dim & 1))
    return fail(AEKV_ERR_VALUE, "%s: rope_dim %d must be even and within [0, %d]", who, rope_dim, d);
  if (pos_sign != 1 && pos_sign != -1) return fail(AEKV_ERR_VALUE, "%s: pos_sign must be +1 or -1", who);
  if (rope_dim > 0 && (!positions || !inv_freq))
    return fail(AEKV_ERR_VALUE, "%s: rope_dim %d needs positions and inv_freq", who, rope_dim);
  if (rows == 0) return AEKV_OK;
  if (!x || !out) return fail(AEKV_ERR_VALUE, "%s: null pointer", who);
  const size_t al = d == 128 ? 4 : 8;
  if (!is_aligned(x, al) || !is_aligned(out, al) || (norm_weight && !is_aligned(norm_weight, 2)))
    return fail(AEKV_ERR_ALIGN, "%s: x and out must be %zu-byte aligned", who, al);
  const int64_t n_vec = rows * heads;
  const int64_t blocks = ceil_div(n_vec, 4);
  if (blocks > 0x7fffffff) return fail(AEKV_ERR_UNSUPPORTED, "%s: %lld vectors exceed the grid", who, (long long)n_vec);
  RopeNormArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.pos = rope_dim > 0 ? positions : nullptr;
  a.inv_freq = inv_freq;
  a.norm = static_cast<const uint16_t*>(norm_weight);
  a.n_vec = n_vec;
  a.heads = heads;
  a.rope_dim = rope_dim;
  a.sign = pos_sign;
  a.eps = eps;
  a.out = static_cast<uint16_t*>(out);
  auto fn = d == 128 ? rope_rmsnorm_kernel<128> : rope_rmsnorm_kernel<256>;
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, as_stream(stream), a);
  return check_launch(who);
}
