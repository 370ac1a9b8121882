// One CSA decode step over TurboQuant-coded caches: indexer scores, exact top-k and sparse sink
// attention over the selected blocks plus the bf16 window.
//
// Reference: aether_2b/serving.py:597-625 (dequantise the index and KV caches, score every block,
// topk(min(256, S)), gather, concat the window, attend with the per-head sink through
// _run_backend :450-467).
//
// Two kernels instead of three: the wide score kernel (idx_mfma_device.h) writes every visible
// key's order key and the 16-key slot maxima; then one workgroup per row selects the row's top-k
// (select_row) and, in the same workgroup, attends the selected blocks and the window
// (attend_main), reading the selection from LDS.  Fusing the two per-row stages removes a kernel
// boundary and the global round trip of the selected indices between them, and lets the
// attention's own loads and set-up run while the select waits on memory; both results are those
// of the separate kernels, which the entry point falls back to outside the fused kernel's limits.
#include <mutex>

#include "idx_mfma_device.h"
#include "quant_attn_device.h"

namespace aekv {
namespace {

constexpr int kFusedThreads = 512;  // 8 waves: the select's 512-thread instance, the 8-wave attention body
constexpr int kFusedCap = 1536;     // select candidates held in LDS
constexpr int kFusedMaxK = 512;     // largest k the 512-thread select sorts outright
constexpr int kFusedMaxW = 128;     // window rows staged in LDS
using FusedLay = qattn::QLay<8, kFusedMaxW>;

// Work that does not depend on the selection is issued before it: the window rows go to LDS with
// direct loads (global_load_lds_dwordx4, lane l -> 16 l bytes past the wave's base, the source
// chunk chosen so that the rows land in the win_chunk layout) and the per-lane query and operand
// constants are built, both overlapping the select's memory rounds.
template <int KV_BITS>
__global__ __launch_bounds__(kFusedThreads) void csa_decode_fused_kernel(idx::MfmaIdxArgs ia, qattn::QAttnMfmaArgs qa,
                                                                       int64_t* __restrict__ out_idx,
                                                                       float* __restrict__ out_score) {
  extern __shared__ __align__(16) unsigned char lds[];
  unsigned char* win_lds = lds + FusedLay::win;
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int W = static_cast<int>(qa.Wt);
  // 4 rows (64 chunks of 16 bytes) per wave instruction
  for (int i = wv; 4 * i < W; i += kFusedThreads / 64) {
    const int r = 4 * i + (lane >> 4);
    if (r < W) {
      const uint16_t* src = qa.win + (static_cast<int64_t>(b) * qa.Wt + r) * qattn::kD + 8 * qattn::win_chunk(r, lane & 15);
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src),
                                       (__attribute__((address_space(3))) void*)(win_lds + 1024 * i), 16, 0, 0);
    }
  }
  qattn::AttnFrags<KV_BITS> f;
  qattn::attend_prologue<KV_BITS>(qa, b, f);
  idx::select_row<kFusedThreads, kFusedCap>(ia, b, out_idx, out_score, reinterpret_cast<int32_t*>(lds + FusedLay::idx));
  __builtin_amdgcn_s_waitcnt(0);  // the window's direct loads (vmcnt) before the barrier in attend_main
  const qattn::RowSources rs = qattn::attend_sources<8>(qa, b, 0, nullptr);
  qattn::attend_main<KV_BITS, 8>(qa, b, 0, lds, f, rs, win_lds);
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
  auto fn = kv_bits == 8 ? csa_decode_fused_kernel<8> : csa_decode_fused_kernel<4>;
  const size_t lds = FusedLay::bytes;
  static std::once_flag once[2];
  std::call_once(once[kv_bits == 8 ? 1 : 0], [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(lds));
  });
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(B)), dim3(kFusedThreads), lds, st, ia, qa, out_idx, out_score);
  return check_launch(who);
}
