// Host side of the matrix-core CSA indexer (kernels in idx_mfma_device.h).
#include "idx_mfma_device.h"

namespace aekv {
namespace idx {

typedef void (*kern_fn)(MfmaIdxArgs);

template <int BITS, int IC>
kern_fn pick_score(int nrb, int tt) {
  if (tt == kScoreTT) {
    switch (nrb) {
      case 1: return idx_mfma_score_kernel<BITS, IC, 1, kScoreTT>;
      case 2: return idx_mfma_score_kernel<BITS, IC, 2, kScoreTT>;
      default: return nullptr;
    }
  }
  switch (nrb) {
    case 1: return idx_mfma_score_kernel<BITS, IC, 1, 1>;
    case 2: return idx_mfma_score_kernel<BITS, IC, 2, 1>;
    case 3: return idx_mfma_score_kernel<BITS, IC, 3, 1>;
    case 4: return idx_mfma_score_kernel<BITS, IC, 4, 1>;
    default: return nullptr;
  }
}

int launch_mfma_score(MfmaIdxArgs& a, const float* q, const float* w, const void* codes, const float* kscale,
                      const float* diag, const int32_t* valid, int64_t B, int64_t T, int64_t S, int IH, int IC,
                      int bits, int k, int mode, void* ws, hipStream_t st, const char* who) {
  a = MfmaIdxArgs{};
  a.T = T;
  a.q = q;
  a.w = w;
  a.codes = static_cast<const uint8_t*>(codes);
  a.kscale = kscale;
  a.diag = diag;
  a.valid = valid;
  a.S = S;
  a.IH = IH;
  a.k = k;
  a.mode = mode;
  a.wscale = wht_scale(IC);
  const WsLayout l = layout(B, S);
  char* base = static_cast<char*>(ws);
  a.keys = reinterpret_cast<uint32_t*>(base + l.keys);
  a.smax = reinterpret_cast<uint32_t*>(base + l.smax);
  a.ms = static_cast<int64_t>(align_up((static_cast<size_t>(S) + 15) / 16, 4));
  a.ks = static_cast<int64_t>(align_up(static_cast<size_t>(S), 16));

  const int nrb = (IH + 3) / 4;
  // prefill rows (T > 1 targets per key row) share each key group kScoreTT rows at a time
  const int tt = (T >= kScoreTT && nrb <= 2) ? kScoreTT : 1;
  kern_fn score = nullptr;
  if (bits == 8) score = IC == 64 ? pick_score<8, 64>(nrb, tt) : pick_score<8, 128>(nrb, tt);
  else score = IC == 64 ? pick_score<4, 64>(nrb, tt) : pick_score<4, 128>(nrb, tt);
  if (!score) return fail(AEKV_ERR_UNSUPPORTED, "%s: no matrix-core indexer for IH=%d IC=%d", who, IH, IC);
  // workgroup rows: one per row, or one per kScoreTT targets of a key row
  const int64_t n_y = tt == 1 ? B : (B / T) * ceil_div(T, static_cast<int64_t>(tt));
  // slot-group size of the score kernel and groups per wave: enough workgroups to fill the chip
  // (~2048), at most 16 groups per wave
  const int64_t group_keys = 64 * score_spw(bits, IC, tt);
  const int64_t groups_per_row = ceil_div(S, group_keys);
  int64_t gpw = (n_y * groups_per_row) / (4 * kScoreTargetWG);
  gpw = std::min<int64_t>(16, std::max<int64_t>(1, gpw));
  a.gpw = static_cast<int>(gpw);
  const int64_t n_score = ceil_div(groups_per_row, 4 * gpw);
  if (B > 65535 || n_score > 0x7fffffff)
    return fail(AEKV_ERR_UNSUPPORTED, "%s: B=%lld S=%lld exceed the launch grid", who, static_cast<long long>(B),
                static_cast<long long>(S));
  hipLaunchKernelGGL(score, dim3(static_cast<uint32_t>(n_score), static_cast<uint32_t>(n_y)), dim3(kThreads), 0, st,
                     a);
  return check_launch(who);
}

}  // namespace idx

using namespace idx;

size_t mfma_indexer_workspace(int64_t B, int64_t S, int32_t k) {
  (void)k;
  return layout(B, S).total;
}

bool mfma_indexer_supported(int IH, int IC, int k, int64_t S) {
  // S >= 1: out-of-range lanes of the score loop read key 0's codes and scale.
  return IH >= 1 && IH <= 4 * kMaxNrb && (IC == 64 || IC == 128) && k >= 1 && k <= kMaxMfmaK && S >= 1 &&
         S <= kMaxKeys;
}

int launch_mfma_indexer(const float* q, const float* w, const void* codes, const float* kscale, const float* diag,
                        const int32_t* valid, int64_t B, int64_t T, int64_t S, int IH, int IC, int bits, int k,
                        int mode, void* ws, int64_t* out_idx, float* out_score, hipStream_t st, const char* who) {
  MfmaIdxArgs a{};
  if (int rc = launch_mfma_score(a, q, w, codes, kscale, diag, valid, B, T, S, IH, IC, bits, k, mode, ws, st, who))
    return rc;
  const uint32_t by = static_cast<uint32_t>(B);
  // rows of at most 16384 keys load 2 (512 threads) or 1 (1024 threads) slot columns per thread
  const bool few_slots = slot_cols_fit(S, 512, 2);
  if (B >= 1024 && k <= 512) {
    auto fn = few_slots ? idx_mfma_final_kernel<512, 1536, 2> : idx_mfma_final_kernel<512, 1536, kHistBins / 512>;
    hipLaunchKernelGGL(fn, dim3(by), dim3(512), 0, st, a, out_idx, out_score);
  } else {
    auto fn = few_slots ? idx_mfma_final_kernel<kSelThreads, kCandCap, 1>
                        : idx_mfma_final_kernel<kSelThreads, kCandCap, kHistBins / kSelThreads>;
    hipLaunchKernelGGL(fn, dim3(by), dim3(kSelThreads), 0, st, a, out_idx, out_score);
  }
  return check_launch(who);
}

}  // namespace aekv
