// One CSA decode step over TurboQuant-coded caches: indexer scores, exact top-k and sparse sink
// attention over the selected blocks plus the bf16 window.
//
// Reference: aether_2b/serving.py:597-625 (dequantise the index and KV caches, score every block,
// topk(min(256, S)), gather, concat the window, attend with the per-head sink through
// _run_backend :450-467).
//
// Two kernels instead of three: the wide score kernel (idx_mfma_device.h) writes every visible
// key's order key and the 16-key slot maxima; then one workgroup per row selects the row's top-k
// (select_row) and, in the same workgroup, attends the window and the selected blocks.  The window
// does not depend on the selection: each wave requests its 16 window rows while the select waits
// for its slot maxima (after them: loads complete in order), and attends them after the select
// while its group of 32 selected blocks (k <= 256) is being gathered, so that neither the select
// nor the gather waits for it.  Fusing
// the two per-row stages also removes a kernel boundary and the global round trip of the selected
// indices between them; the selection is that of the separate kernels, and the attention that of
// the separate attention kernel up to the order in which the sources are summed (the entry point
// runs the separate kernels outside the fused kernel's limits).
#include <mutex>

#include "idx_mfma_device.h"
#include "quant_attn_device.h"

namespace aekv {
namespace {

constexpr int kFusedThreads = 512;  // 8 waves: the select's 512-thread instance, the 8-wave attention body
constexpr int kFusedCap = 1536;     // select candidates held in LDS
constexpr int kFusedMaxK = 512;     // largest k the 512-thread select sorts outright
constexpr int kFusedMaxW = 128;     // window rows: 16 per wave
using FusedLay = qattn::QLay<8>;

template <int KV_BITS, int COLS>
__global__ __launch_bounds__(kFusedThreads) void csa_decode_fused_kernel(idx::MfmaIdxArgs ia, qattn::QAttnMfmaArgs qa,
                                                                       int64_t* __restrict__ out_idx,
                                                                       float* __restrict__ out_score) {
  constexpr int NW = kFusedThreads / 64;
  touch_kernargs<sizeof(ia) + sizeof(qa) + 2 * sizeof(void*)>();
  extern __shared__ __align__(16) unsigned char lds[];
  int32_t* sel_lds = reinterpret_cast<int32_t*>(lds + FusedLay::idx);
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, c16 = lane & 15;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = static_cast<int>(qa.Wt);
  // first memory round: the query and diagonal, then the row's visible count (a scalar load: the
  // select's slot ranges wait for it alone), then the select's slot maxima
  const bool has_win = 16 * wv < W;  // wave-uniform
  const bool wok = 16 * wv + c16 < W;
  qattn::PrologueRaw praw;
  qattn::prologue_loads(qa, b, praw);
  const int64_t nv = idx::visible(ia, b);
  qattn::AttnFrags<KV_BITS> f;
  qattn::AttnState st;
  qattn::attn_state_init(st);
  // While the select waits for its maxima: the wave's window entries 16 wv .. 16 wv + 15 are
  // requested (block 0 of a group, entries past W no source) and the query fragments built.  The
  // window rows are requested after the maxima because loads complete in order: ahead of them they
  // delay the select, and they are only attended after it, while the wave's first group of
  // selected rows is requested.
  qattn::GroupIn<KV_BITS> win_in;
  bool built = false;
  auto build = [&]() {
    qattn::window_fetch<KV_BITS>(qa, b, 16 * wv + c16, win_in);
    qattn::prologue_build<KV_BITS>(qa, praw, f);
    built = true;
  };
  const uint32_t kk = idx::select_row<kFusedThreads, kFusedCap, COLS>(ia, b, nv, out_idx, out_score, sel_lds, build);
  if (!built) build();  // a row with no visible block skips the select's memory rounds
  __syncthreads();      // sel_lds
  auto window = [&]() {
    const bool okm[2] = {wok, false};
    qattn::group_consume<KV_BITS>(qa, f, win_in, st, okm);
  };
  // the selected blocks, in the same state: wave w takes groups w, w + NW, ...
  const int n_groups = static_cast<int>((kk + qattn::kGroup - 1) / qattn::kGroup);
  bool win_pending = has_win;  // wave-uniform
#pragma unroll 1
  for (int G = wv; G < n_groups; G += NW) {
    qattn::SrcRef src[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int si = G * qattn::kGroup + 16 * kb + c16;
      const int32_t blk = si < static_cast<int>(kk) ? sel_lds[si] : -1;
      src[kb].kind = blk >= 0 ? 1 : 0;
      src[kb].at = blk;
    }
    qattn::GroupIn<KV_BITS, false> in;
    qattn::group_fetch<KV_BITS, false>(qa, b, src, nullptr, in);
    if (win_pending) {
      window();
      win_pending = false;
    }
    qattn::group_consume<KV_BITS, false>(qa, f, in, st);
  }
  if (win_pending) window();  // a wave without a selected group
  qattn::attend_finish<NW>(qa, b, 0, lds, st, f.sink, f.neg);
}

}  // namespace
}  // namespace aekv

using namespace aekv;

extern "C" size_t aekv_csa_decode_workspace_size(int64_t B, int64_t S, int32_t k, int64_t H, int64_t D, int64_t W) {
  const size_t wi = align_up(aekv_csa_indexer_workspace_size(B, S, k), 256);
  return wi + aekv_quant_attention_workspace_size(B, H, D, k, W);
}

extern "C" int aekv_csa_decode_quant(const float* index_q, const float* index_weight, const void* index_codes,
                                     const float* index_scale, const float* index_diag, const int32_t* valid, int64_t B,
                                     int64_t S, int32_t IH, int32_t IC, int32_t index_bits, int32_t k, int32_t mode,
                                     const void* q, const void* kv_codes, const float* kv_scale, const void* window,
                                     const float* sink, const float* kv_diag, int64_t H, int64_t D, int64_t W,
                                     int32_t kv_bits, float softmax_scale, void* ws, size_t ws_bytes, int64_t* out_idx,
                                     float* out_score, void* out, void* stream) {
  const char* who = "aekv_csa_decode_quant";
  if (int rc = validate_quant_rows(index_q, index_weight, index_codes, index_scale, index_diag, B, 1, S, IH, IC,
                                   index_bits, k, mode, ws, ws_bytes, out_idx, who))
    return rc;
  if (kv_bits != 4 && kv_bits != 8) return fail(AEKV_ERR_VALUE, "bits must be 4 or 8, got %d", kv_bits);
  if (!is_pow2(D)) return fail(AEKV_ERR_VALUE, "WHT requires last dim to be a power of 2, got %lld", (long long)D);
  if (H <= 0 || W < 0) return fail(AEKV_ERR_SHAPE, "%s: bad sizes H=%lld W=%lld", who, (long long)H, (long long)W);
  const size_t wi = align_up(aekv_csa_indexer_workspace_size(B, S, k), 256);
  const size_t need = aekv_csa_decode_workspace_size(B, S, k, H, D, W);
  if (B > 0 && ws_bytes < need)
    return fail(AEKV_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who, need, ws_bytes);
  if (B == 0) return AEKV_OK;
  if (!q || !sink || !kv_diag || !out || !kv_codes || !kv_scale || (W > 0 && !window))
    return fail(AEKV_ERR_VALUE, "%s: null pointer", who);
  const hipStream_t st = as_stream(stream);
  const bool fused = use_specialised_codec() && mfma_indexer_supported(IH, IC, k, S) && k <= kFusedMaxK &&
                     quant_attn_mfma_supported(H, D) && W <= kFusedMaxW && B <= 65535 &&
                     is_aligned(q, 16) && is_aligned(out, 8) && is_aligned(kv_diag, 16) && is_aligned(kv_codes, 16) &&
                     (W == 0 || is_aligned(window, 16));
  if (!fused) {
    if (int rc = aekv_csa_indexer_topk_quant(index_q, index_weight, index_codes, index_scale, index_diag, valid, B, S,
                                             IH, IC, index_bits, k, mode, ws, wi, out_idx, out_score, stream))
      return rc;
    return aekv_quant_sink_attention(q, kv_codes, kv_scale, out_idx, window, sink, kv_diag, B, H, D, S, k, W, kv_bits,
                                     softmax_scale, static_cast<char*>(ws) + wi, ws_bytes - wi, out, stream);
  }
  idx::MfmaIdxArgs ia{};
  if (int rc = idx::launch_mfma_score(ia, index_q, index_weight, index_codes, index_scale, index_diag, valid, B, 1, S,
                                      IH, IC, index_bits, k, mode, ws, st, who))
    return rc;
  qattn::QAttnMfmaArgs qa{};
  qa.q = static_cast<const uint16_t*>(q);
  qa.codes = static_cast<const uint8_t*>(kv_codes);
  qa.scale = kv_scale;
  qa.sel = out_idx;  // marks the selected-blocks mode; the indices themselves are read from LDS
  qa.win = static_cast<const uint16_t*>(window);
  qa.sink = sink;
  qa.diag = kv_diag;
  qa.T = 1;
  qa.Wt = W;
  qa.S = S;
  qa.K = k;
  qa.n_comp = k;
  qa.n_src = k + W;
  qa.H = static_cast<int>(H);
  qa.n_split = 1;
  qa.split_src = qattn::kSplitSrc;
  qa.sm_scale = softmax_scale;
  qa.wscale = wht_scale(qattn::kD);
  qa.out = static_cast<uint16_t*>(out);
  // rows of at most 16384 keys: the select loads 2 slot columns per thread instead of 8
  constexpr int kWide = idx::kHistBins / kFusedThreads;
  const bool few = idx::slot_cols_fit(S, kFusedThreads, 2);
  auto fn = kv_bits == 8 ? (few ? csa_decode_fused_kernel<8, 2> : csa_decode_fused_kernel<8, kWide>)
                         : (few ? csa_decode_fused_kernel<4, 2> : csa_decode_fused_kernel<4, kWide>);
  const size_t lds = FusedLay::bytes;
  static std::once_flag once[4];
  std::call_once(once[(kv_bits == 8 ? 2 : 0) + (few ? 1 : 0)], [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(lds));
  });
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(B)), dim3(kFusedThreads), lds, st, ia, qa, out_idx, out_score);
  return check_launch(who);
}
