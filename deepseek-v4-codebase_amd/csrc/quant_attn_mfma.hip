// Host side of the decode-step attention over TurboQuant-coded blocks (kernels in
// quant_attn_device.h) and the split combine kernel.
#include <mutex>

#include "quant_attn_device.h"

namespace aekv {
namespace qattn {

// Split combine: M = max(sink, split maxima), L = e^{sink-M} + sum_s e^{m_s-M} l_s,
// out = sum_s e^{m_s-M} acc_s / L.  The per-head factors e^{m_s-M} / L go to LDS first (one load
// round for every split's statistics), then each output sums its splits' partials, all loads of a
// thread issued together: two dependent memory rounds per row whatever the split count.
constexpr int kMaxCombineSplits = 256;
__global__ __launch_bounds__(kThreads) void quant_attn_mfma_combine_kernel(QAttnMfmaArgs a) {
  __shared__ float st[kMaxCombineSplits * 16 * 2];  // [split][head][m, l]
  __shared__ float fac[kMaxCombineSplits * 16];     // [split][head] e^{m_s - M} / L
  const int64_t b = blockIdx.x;
  const int H = a.H, ns = a.n_split;
  const float* part = a.part + b * ns * H * (kD + 2);
  for (int i = threadIdx.x; i < ns * H; i += kThreads) {
    const float* ps = part + static_cast<int64_t>(i) * (kD + 2);
    st[2 * i] = ps[0];
    st[2 * i + 1] = ps[1];
  }
  __syncthreads();
  if (threadIdx.x < H) {
    const int h = threadIdx.x;
    const float sk = a.sink[h];
    float M = sk;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, st[2 * (s * H + h)]);
    float L = __expf(sk - M);
    for (int s = 0; s < ns; ++s) {
      const float ms = st[2 * (s * H + h)];
      const float f = ms == kNegInf ? 0.0f : __expf(ms - M);
      fac[s * H + h] = f;
      L = fmaf(f, st[2 * (s * H + h) + 1], L);
    }
    const float r = 1.0f / L;
    for (int s = 0; s < ns; ++s) fac[s * H + h] *= r;
  }
  __syncthreads();
  // thread -> (head, 4 consecutive dims); the splits' partials are independent loads
  for (int p = threadIdx.x; p < H * (kD / 4); p += kThreads) {
    const int h = p / (kD / 4), d4 = 4 * (p % (kD / 4));
    f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
    for (int s = 0; s < ns; ++s) {
      const float* ps = part + static_cast<int64_t>(s * H + h) * (kD + 2) + 2 + d4;
      const float f = fac[s * H + h];
      acc = f32x4_t{fmaf(f, ps[0], acc[0]), fmaf(f, ps[1], acc[1]), fmaf(f, ps[2], acc[2]), fmaf(f, ps[3], acc[3])};
    }
    const uint2 v = make_uint2(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]));
    *reinterpret_cast<uint2*>(a.out + (b * H + h) * kD + d4) = v;
  }
}


}  // namespace qattn

using namespace qattn;

// Sources per workgroup: kSplitSrc, halved (down to kMinSplitSrc) while the grid has fewer
// than kTargetWG workgroups, so that few long rows still spread over the chip.  A row
// with more sources than that takes one workgroup per piece plus the split combine.
int64_t split_sources(int64_t rows, int64_t n_src) {
  int64_t s = kSplitSrc;
  while (s > kMinSplitSrc && rows * ceil_div(std::max<int64_t>(n_src, 1), s) < kTargetWG) s >>= 1;
  return s;
}

bool quant_attn_mfma_supported(int64_t H, int64_t D) { return D == kD && H >= 1 && H <= 16; }

bool quant_attn_mfma_fits(int64_t rows, int64_t n_src) {
  return rows <= 65535 && (n_src <= 0 || ceil_div(n_src, split_sources(rows, n_src)) <= kMaxCombineSplits);
}

size_t quant_attn_mfma_workspace(int64_t B, int64_t H, int64_t n_src) {
  const int64_t n_split = n_src > 0 ? ceil_div(n_src, split_sources(B, n_src)) : 1;
  return n_split > 1 ? align_up(static_cast<size_t>(B * n_split * H * (kD + 2)) * 4, 256) : 0;
}

int launch_quant_attn_mfma_rows(const void* q, const void* codes, const float* scale, const int64_t* sel,
                                const int32_t* vis, const void* window, const int32_t* wstart, const int32_t* wlen,
                                const float* sink, const float* diag, int64_t rows, int64_t T, int64_t H, int64_t S,
                                int64_t K, bool all_blocks, int64_t Wt, int bits, float softmax_scale, void* ws,
                                void* out, hipStream_t st, const char* who) {
  QAttnMfmaArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.codes = static_cast<const uint8_t*>(codes);
  a.scale = scale;
  a.sel = all_blocks ? nullptr : sel;
  a.vis = vis;
  a.win = static_cast<const uint16_t*>(window);
  a.wstart = wstart;
  a.wlen = wlen;
  a.sink = sink;
  a.diag = diag;
  a.T = T;
  a.Wt = Wt;
  a.S = S;
  a.K = K;
  a.n_comp = all_blocks ? S : K;
  a.n_src = a.n_comp + Wt;  // an upper bound of every row's sources
  a.H = static_cast<int>(H);
  a.split_src = static_cast<int>(split_sources(rows, a.n_src));
  const int64_t n_split = a.n_src > 0 ? ceil_div(a.n_src, static_cast<int64_t>(a.split_src)) : 1;
  if (n_split > kMaxCombineSplits || rows > 65535)
    return fail(AEKV_ERR_UNSUPPORTED, "%s: %lld rows x %lld sources exceed the launch grid", who,
                static_cast<long long>(rows), static_cast<long long>(a.n_src));
  a.n_split = static_cast<int>(n_split);
  a.sm_scale = softmax_scale;
  a.wscale = wht_scale(kD);
  a.part = static_cast<float*>(ws);
  a.out = static_cast<uint16_t*>(out);
  // 4 waves per workgroup once the launch has >= 1024 workgroups (prefill rows), else 8
  const bool narrow = rows * n_split >= 1024;
  auto fn = narrow ? (bits == 8 ? quant_attn_mfma_kernel<8, 4> : quant_attn_mfma_kernel<4, 4>)
                   : (bits == 8 ? quant_attn_mfma_kernel<8, 8> : quant_attn_mfma_kernel<4, 8>);
  const size_t lds = narrow ? QLay<4>::bytes : QLay<8>::bytes;
  static std::once_flag once[4];
  std::call_once(once[(bits == 8 ? 2 : 0) + (narrow ? 1 : 0)], [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(lds));
  });
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(n_split), static_cast<uint32_t>(rows)), dim3(narrow ? 256 : kThreads),
                     lds, st, a);
  if (int rc = check_launch(who)) return rc;
  if (n_split > 1) {
    hipLaunchKernelGGL(quant_attn_mfma_combine_kernel, dim3(static_cast<uint32_t>(rows)), dim3(kThreads), 0, st, a);
    return check_launch(who);
  }
  return AEKV_OK;
}

int launch_quant_attn_mfma(const void* q, const void* codes, const float* scale, const int64_t* sel,
                           const void* window, const float* sink, const float* diag, int64_t B, int64_t H, int64_t S,
                           int64_t K, bool all_blocks, int64_t W, int bits, float softmax_scale, void* ws,
                           void* out, hipStream_t st, const char* who) {
  return launch_quant_attn_mfma_rows(q, codes, scale, sel, nullptr, window, nullptr, nullptr, sink, diag, B, 1, H, S,
                                     K, all_blocks, W, bits, softmax_scale, ws, out, st, who);
}

}  // namespace aekv
