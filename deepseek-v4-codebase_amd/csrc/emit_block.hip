// Block emission: softmax-pool a compressed block's token entries, RoPE at the block position,
// RMSNorm, and TurboQuant-encode the result into its slot of a code ring — one kernel per block.
//
// Reference: aether_2b/serving.py:495-505 (_hca_emit) and :557-576 (_emit_csa_block: main part
// with RoPE + kv_norm, index part without), modeling.py:122-155 (apply_rope), :32-41 (RMSNorm),
// turbo_quant.py:127-166 (encode).  The reference runs these as separate torch ops over bf16
// tensors; this kernel keeps their rounding points:
//   zz  = bf16(z + bias)                         (bias optional: the CSA per-slot biases)
//   w_m = bf16(exp(zz_m - max) * (1 / sum_m exp(zz_m - max)))      fp32, sums in m order
//   x   = bf16(sum_m float(bf16(w_m * c_m)))                        fp32 sum in m order
//   RoPE on the last rope_dim dims, pairs (2i, 2i+1), cos/sin = bf16(cos/sin(fp32(pos) * f_i)):
//     even bf16(bf16(a cos) + bf16(-b sin)), odd bf16(bf16(b cos) + bf16(a sin))
//   RMSNorm: r = 1 / sqrt(mean(x^2) + eps) in fp32, y = bf16((x * r) * w)
// and then encodes y exactly as PolarQuant.encode would (the same per-lane sequence as the
// generic encode kernel).  Only the library exp/cos/sin/sqrt and the order of the mean's sum can
// differ from torch's CPU kernels, i.e. an ulp of fp32 before the bf16 roundings.
//
// One workgroup of D threads per row; thread d owns dim d through the pooling, RoPE (the pair
// partner is lane d ^ 1) and RMSNorm (wave sums + LDS); the pooled vector then goes through LDS to
// the first D/8 lanes, which encode it (8 elements per lane).
#include "tq_device.h"

namespace aekv {
namespace {

struct EmitArgs {
  const uint16_t* c;      // [B, L, D] bf16
  const uint16_t* z;      // [B, L, D] bf16
  const uint16_t* bias;   // [L, D] bf16 or null
  const int64_t* pos;     // [B] or null (no RoPE)
  const float* inv_freq;  // [rope_dim / 2]
  const uint16_t* norm;   // [D] bf16 or null (no RMSNorm)
  const float* diag;      // [D]
  int64_t L, row_stride;
  int rope_dim;
  float eps, wscale;
  uint8_t* codes;         // [B, row_stride, D or D/2]: the block goes to row b, slot 0 of this view
  float* scale;           // [B, row_stride]
  uint16_t* vec;          // [B, D] bf16 or null: the pooled, normalised vector before encoding
};

__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(pack_bf16x2(v, 0.0f) & 0xFFFFu); }

template <int D, int BITS>
__global__ __launch_bounds__(D) void emit_block_kernel(EmitArgs a) {
  constexpr int EPL = 8, LPV = D / EPL;
  constexpr int NW = D / 64;
  __shared__ float xs[D];
  __shared__ float red[NW];
  const int64_t b = blockIdx.x;
  const int d = threadIdx.x, lane = d & 63;
  const uint16_t* zr = a.z + b * a.L * D + d;
  const uint16_t* cr = a.c + b * a.L * D + d;
  auto zval = [&](int64_t m) {
    float zz = bf16_to_f32(zr[m * D]);
    if (a.bias) zz = bf16r(zz + bf16_to_f32(a.bias[m * D + d]));
    return zz;
  };
  // softmax over the L entries of dim d, then the weighted sum (three passes, L2-resident rows)
  float mx = -__builtin_inff();
  for (int64_t m = 0; m < a.L; ++m) mx = fmaxf(mx, zval(m));
  float sum = 0.0f;
  for (int64_t m = 0; m < a.L; ++m) sum += expf(zval(m) - mx);
  const float inv = 1.0f / sum;
  float acc = 0.0f;
  for (int64_t m = 0; m < a.L; ++m) {
    const float w = bf16r(expf(zval(m) - mx) * inv);
    acc += bf16r(w * bf16_to_f32(cr[m * D]));
  }
  float x = bf16r(acc);
  // RoPE on the last rope_dim dims: the pair partner is lane d ^ 1
  if (a.pos) {
    const int r0 = D - a.rope_dim;
    const float partner = xor_lane<1>(x);
    if (d >= r0) {
      const int i = (d - r0) >> 1;
      const float ang = static_cast<float>(a.pos[b]) * a.inv_freq[i];
      const float cs = bf16r(cosf(ang)), sn = bf16r(sinf(ang));
      x = (d & 1) ? bf16r(bf16r(x * cs) + bf16r(partner * sn)) : bf16r(bf16r(x * cs) + bf16r(-partner * sn));
    }
  }
  // RMSNorm
  if (a.norm) {
    float ss = wave_sum(x * x);
    if (lane == 0) red[d >> 6] = ss;
    __syncthreads();
    ss = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) ss += red[w];
    const float r = 1.0f / sqrtf(ss / static_cast<float>(D) + a.eps);
    x = bf16r((x * r) * bf16_to_f32(a.norm[d]));
  }
  if (a.vec) a.vec[b * D + d] = static_cast<uint16_t>(pack_bf16x2(x, 0.0f) & 0xFFFFu);
  xs[d] = x;
  __syncthreads();
  // encode: lanes 0 .. LPV-1 of wave 0 hold elements 8 sub .. 8 sub + 7 (every lane of the wave
  // takes part in the exchanges; only those lanes store)
  if (d < 64) {
    const int sub = lane % LPV;
    float v[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) v[e] = xs[sub * EPL + e] * a.diag[sub * EPL + e];  // x.float() * diag
    float m;
    constexpr int NB = BITS == 8 ? EPL : EPL / 2;
    const Bytes<NB> w = encode_lane<BITS, D, true>(v, sub, a.wscale, &m);
    if (lane < LPV) {
      *reinterpret_cast<Bytes<NB>*>(a.codes + b * a.row_stride * (BITS == 8 ? D : D / 2) + sub * NB) = w;
      if (sub == 0) a.scale[b * a.row_stride] = m / (BITS == 8 ? 127.0f : 7.0f);
    }
  }
}

using emit_fn = void (*)(EmitArgs);

emit_fn pick_emit(int d, int bits) {
  if (d == 64) return bits == 8 ? emit_block_kernel<64, 8> : emit_block_kernel<64, 4>;
  if (d == 128) return bits == 8 ? emit_block_kernel<128, 8> : emit_block_kernel<128, 4>;
  return nullptr;
}

}  // namespace
}  // namespace aekv

using namespace aekv;

extern "C" int aekv_emit_block(const void* c, const void* z, const void* z_bias, int64_t B, int64_t len, int32_t d,
                               int32_t rope_dim, const int64_t* positions, const float* inv_freq,
                               const void* norm_weight, float eps, int32_t bits, const float* diag, void* out_codes,
                               float* out_scale, int64_t out_row_stride, void* out_vec, void* stream) {
  const char* who = "aekv_emit_block";
  if (bits != 4 && bits != 8) return fail(AEKV_ERR_VALUE, "bits must be 4 or 8, got %d", bits);
  if (d != 64 && d != 128) return fail(AEKV_ERR_UNSUPPORTED, "%s: head dim %d (64 or 128 supported)", who, d);
  if (B < 0 || len < 1) return fail(AEKV_ERR_SHAPE, "%s: B=%lld len=%lld", who, (long long)B, (long long)len);
  if (out_row_stride < 1) return fail(AEKV_ERR_SHAPE, "%s: out_row_stride %lld < 1", who, (long long)out_row_stride);
  if (rope_dim < 0 || rope_dim > d || (rope_dim & 1))
    return fail(AEKV_ERR_VALUE, "%s: rope_dim %d must be even and within [0, %d]", who, rope_dim, d);
  if (rope_dim > 0 && (!positions || !inv_freq))
    return fail(AEKV_ERR_VALUE, "%s: rope_dim %d needs positions and inv_freq", who, rope_dim);
  if (B == 0) return AEKV_OK;
  if (!c || !z || !diag || !out_codes || !out_scale) return fail(AEKV_ERR_VALUE, "%s: null pointer", who);
  if (!is_aligned(c, 2) || !is_aligned(z, 2) || !is_aligned(out_scale, 4) || !is_aligned(diag, 4))
    return fail(AEKV_ERR_ALIGN, "%s: misaligned pointer", who);
  const size_t nb = bits == 8 ? 8 : 4;  // code bytes a lane stores
  if (!is_aligned(out_codes, nb)) return fail(AEKV_ERR_ALIGN, "%s: out_codes must be %zu-byte aligned", who, nb);
  if (B > 0x7fffffff) return fail(AEKV_ERR_UNSUPPORTED, "%s: B=%lld exceeds the grid", who, (long long)B);
  EmitArgs a{};
  a.c = static_cast<const uint16_t*>(c);
  a.z = static_cast<const uint16_t*>(z);
  a.bias = static_cast<const uint16_t*>(z_bias);
  a.pos = rope_dim > 0 ? positions : nullptr;
  a.inv_freq = inv_freq;
  a.norm = static_cast<const uint16_t*>(norm_weight);
  a.diag = diag;
  a.L = len;
  a.row_stride = out_row_stride;
  a.rope_dim = rope_dim;
  a.eps = eps;
  a.wscale = wht_scale(d);
  a.codes = static_cast<uint8_t*>(out_codes);
  a.scale = out_scale;
  a.vec = static_cast<uint16_t*>(out_vec);
  hipLaunchKernelGGL(pick_emit(d, bits), dim3(static_cast<uint32_t>(B)), dim3(d), 0, as_stream(stream), a);
  return check_launch(who);
}
