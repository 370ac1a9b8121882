// Host side of the decode-step attention over TurboQuant-coded blocks (kernels in
// quant_attn_device.h) and the split combine kernel.
#include <mutex>

#include "quant_attn_device.h"

namespace aekv {
namespace qattn {

constexpr int kMaxCombineSplits = 256;  // most source pieces per row

// Split combine: M = max(sink, split maxima), L = e^{sink-M} + sum_s e^{m_s-M} l_s,
// out = sum_s e^{m_s-M} acc_s / L (the sink counted once, aether_pipeline/serving.py:125-129).  32
// threads per (row, head), 4 dims each; the splits' (m, l, acc) are loaded in chunks of 8 whose
// loads are all issued together (the first chunk's with the sink's) and merged online, so a row
// takes one memory round per 8 splits.  Workgroups of kCombineThreads (two (row, head) pairs): a
// decode step's few hundred pairs then spread over as many CUs, instead of queueing their loads on
// a few.  The arguments are plain scalars, which the dispatch preloads into registers (this file
// is built with kernel-argument preloading), so the first loads do not wait for the argument
// block.
constexpr int kCombineThreads = 64;
__global__ __launch_bounds__(kCombineThreads) void quant_attn_mfma_combine_kernel(const float* __restrict__ part,
                                                                                  const float* __restrict__ sink,
                                                                                  uint16_t* __restrict__ out,
                                                                                  int rows_heads, int H, int ns) {
  constexpr int kChunk = 8;
  const int rh = static_cast<int>(blockIdx.x) * (kCombineThreads / 32) + (static_cast<int>(threadIdx.x) >> 5);
  if (rh >= rows_heads) return;
  const int b = rh / H, h = rh - b * H, j = threadIdx.x & 31;
  // split s of (row b, head h) at prow + s H kPartStride; a split past ns reads split 0 (always
  // present) and is replaced by the empty state (max -inf, sum 0, acc 0)
  const float* prow = part + (static_cast<int64_t>(b) * ns * H + h) * kPartStride;
  float m[kChunk], l[kChunk];
  f32x4_t o[kChunk];
  // the chunk's loads all precede the empty asm that takes their values, so every load is issued
  // before the first wait (the compiler would otherwise move loads into the branches that use
  // them, each with its own wait)
  auto load_chunk = [&](const int s0, float* sk) {
    float2 ml[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const float* ps = prow + static_cast<int64_t>(s0 + i < ns ? s0 + i : 0) * H * kPartStride;
      ml[i] = *reinterpret_cast<const float2*>(ps);
      o[i] = *reinterpret_cast<const f32x4_t*>(ps + 4 + 4 * j);
    }
    if (sk) *sk = sink[h];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) asm volatile("" : "+v"(ml[i].x), "+v"(ml[i].y), "+v"(o[i]));
    if (sk) asm volatile("" : "+v"(*sk));
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const bool in = s0 + i < ns;
      m[i] = in ? ml[i].x : kNegInf;
      l[i] = in ? ml[i].y : 0.0f;
      o[i] = in ? o[i] : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  float sk;
  load_chunk(0, &sk);
  float M = sk, den = sk == kNegInf ? 0.0f : 1.0f;
  f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < ns; s0 += kChunk) {
    if (s0 > 0) load_chunk(s0, nullptr);
    float cm = M;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) cm = fmaxf(cm, m[i]);
    if (cm == kNegInf) continue;  // nothing yet (no sink, no source)
    const float r = M == kNegInf ? 0.0f : __expf(M - cm);
    den *= r;
    acc *= r;
    M = cm;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const float f = m[i] == kNegInf ? 0.0f : __expf(m[i] - M);
      den = fmaf(f, l[i], den);
      acc = f32x4_t{fmaf(f, o[i][0], acc[0]), fmaf(f, o[i][1], acc[1]), fmaf(f, o[i][2], acc[2]), fmaf(f, o[i][3], acc[3])};
    }
  }
  const float r = den > 0.0f ? 1.0f / den : 0.0f;
  *reinterpret_cast<uint2*>(out + static_cast<int64_t>(rh) * kD + 4 * j) =
      make_uint2(pack_bf16x2(acc[0] * r, acc[1] * r), pack_bf16x2(acc[2] * r, acc[3] * r));
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
  return n_split > 1 ? align_up(static_cast<size_t>(B * n_split * H * kPartStride) * 4, 256) : 0;
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
  a.n_comp = all_blocks ? std::min(K, S) : K;
  a.n_src = a.n_comp + Wt;  // an upper bound of every row's sources
  a.H = static_cast<int>(H);
  // decode rows over every block without counts take the dense kernel (its buffer ranges, one cache
  // row's codes and window entries, must stay below 2^31 bytes)
  const bool dense = T == 1 && all_blocks && !vis && !wstart && !wlen &&
                     S * (bits == 8 ? kD : kD / 2) < (int64_t{1} << 31) && Wt * kD * 2 < (int64_t{1} << 31);
  a.split_src = static_cast<int>(split_sources(rows, a.n_src));
  const int64_t n_split = a.n_src > 0 ? ceil_div(a.n_src, static_cast<int64_t>(a.split_src)) : 1;
  if (n_split > kMaxCombineSplits || rows > 65535)
    return fail(AEKV_ERR_UNSUPPORTED, "%s: %lld rows x %lld sources exceed the launch grid", who,
                static_cast<long long>(rows), static_cast<long long>(a.n_src));
  a.n_split = static_cast<int>(n_split);
  if (n_split > 1 && (!ws || !is_aligned(ws, 16)))
    return fail(AEKV_ERR_ALIGN, "%s: the split workspace must be 16-byte aligned", who);
  a.sm_scale = softmax_scale;
  a.wscale = wht_scale(kD);
  a.part = static_cast<float*>(ws);
  a.out = static_cast<uint16_t*>(out);
  // 4 waves per workgroup once the launch has >= 1024 workgroups (prefill rows), else 8
  const bool narrow = !dense && rows * n_split >= 1024;
  auto fn = dense ? (bits == 8 ? quant_attn_dense_kernel<8> : quant_attn_dense_kernel<4>)
          : narrow ? (bits == 8 ? quant_attn_mfma_kernel<8, 4> : quant_attn_mfma_kernel<4, 4>)
                   : (bits == 8 ? quant_attn_mfma_kernel<8, 8> : quant_attn_mfma_kernel<4, 8>);
  const size_t lds = narrow ? QLay<4>::bytes : QLay<8>::bytes;
  static std::once_flag once[6];
  std::call_once(once[(bits == 8 ? 3 : 0) + (dense ? 2 : narrow ? 1 : 0)], [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(lds));
  });
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(n_split), static_cast<uint32_t>(rows)), dim3(narrow ? 256 : kThreads),
                     lds, st, a);
  if (int rc = check_launch(who)) return rc;
  if (n_split > 1) {
    const int64_t n_wg = ceil_div(rows * H, kCombineThreads / 32);
    hipLaunchKernelGGL(quant_attn_mfma_combine_kernel, dim3(static_cast<uint32_t>(n_wg)), dim3(kCombineThreads), 0, st,
                       static_cast<const float*>(a.part), a.sink, a.out, static_cast<int>(rows * H), a.H, a.n_split);
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
