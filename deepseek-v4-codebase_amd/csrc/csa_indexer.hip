// CSA lightning indexer + exact top-k for gfx950.
//
// Reference: aether_2b/modeling.py:604-616 (softplus rule, top-k), aether_2b/serving.py:616-621
// (raw-weight rule used in serving decode), aether_kernels/sparse_attention.py:45-67 and
// aether_kernels/csrc/csa_indexer_cuda.cu:21-110 (fp32 API; relu-on-weight rule).
//
// Two kernels per call:
//   1. idx_score_chunk: grid (chunks, B).  A workgroup scores kChunk keys of one row into LDS and
//      keeps the chunk's k best under the total order (score desc, index asc) with an LDS radix
//      select.  Candidates go to the workspace.
//   2. idx_merge: grid B.  Radix-selects the k best of the row's candidates, bitonic-sorts them in
//      LDS and writes int64 indices (+ fp32 scores).
// The total order is strict, so every global top-k element is in its chunk's top-k and the
// two-level select is exact.  Ties in score go to the lower index (torch.topk leaves tie order
// unspecified; only the selected set is compared).
//
// Quantised keys are scanned in the rotated domain: q.k_j = scale_j * (WHT(diag*q) . codes_j)
// (the WHT is orthogonal and symmetric; turbo_quant.py:208-209), and since scale_j > 0,
// relu(scale_j * x) = scale_j * relu(x).
#include <algorithm>
#include <mutex>

#include "aekv_common.h"

namespace aekv {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 4096;
constexpr int kMaxK = 2048;
constexpr int kMaxIH = 64;
constexpr int kMaxIC = 256;

enum KeyFmt { kKeyF32 = 0, kKeyQ8 = 8, kKeyQ4 = 4 };

__device__ __forceinline__ float softplus_f32(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Block-wide inclusive scan (sum) of one uint32 per thread, 256 threads.  `tmp` holds 256 words.
__device__ uint32_t block_inclusive_scan(uint32_t v, uint32_t* tmp) {
  const int t = threadIdx.x;
  tmp[t] = v;
  __syncthreads();
#pragma unroll
  for (int off = 1; off < kThreads; off <<= 1) {
    const uint32_t add = t >= off ? tmp[t - off] : 0u;
    __syncthreads();
    tmp[t] += add;
    __syncthreads();
  }
  const uint32_t r = tmp[t];
  __syncthreads();
  return r;
}

// Finds the k-th largest order key T among keys[0..n) (n > k > 0) and the number of keys > T.
// `get(i)` returns key i.  hist: 256 words, tmp: 256 words of LDS.
template <typename Get>
__device__ void radix_threshold(Get get, int n, int k, uint32_t* hist, uint32_t* tmp, uint32_t* bcast,
                                uint32_t& T, int& n_gt) {
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[threadIdx.x] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kThreads) {
      const uint32_t u = get(i);
      if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
    }
    __syncthreads();
    // suffix counts: thread t gets sum_{d >= t} hist[d]  (scan over reversed digits)
    const uint32_t mine = hist[255 - threadIdx.x];
    const uint32_t incl = block_inclusive_scan(mine, tmp);  // = sum_{d >= 255-t} hist[d]
    const uint32_t excl = incl - mine;                      // = sum_{d > 255-t} hist[d]
    if (excl < static_cast<uint32_t>(remaining) && incl >= static_cast<uint32_t>(remaining)) {
      bcast[0] = 255u - threadIdx.x;
      bcast[1] = excl;
    }
    __syncthreads();
    const uint32_t dgt = bcast[0];
    remaining -= static_cast<int>(bcast[1]);
    prefix |= dgt << shift;
    mask |= 255u << shift;
    __syncthreads();
  }
  T = prefix;
  n_gt = k - remaining;
}

// Writes the k best of keys[0..n) under (key desc, position asc) into (out_key, out_idx) using
// stable block-wide compaction in position order: first all keys > T, then keys == T.
template <typename Get, typename Idx>
__device__ int select_compact(Get get, Idx idx_of, int n, int k, uint32_t* hist, uint32_t* tmp, uint32_t* bcast,
                              uint32_t* out_key, int32_t* out_idx) {
  if (n <= k) {
    for (int i = threadIdx.x; i < n; i += kThreads) {
      out_key[i] = get(i);
      out_idx[i] = idx_of(i);
    }
    return n;
  }
  uint32_t T;
  int n_gt;
  radix_threshold(get, n, k, hist, tmp, bcast, T, n_gt);
  const int per = (n + kThreads - 1) / kThreads;
  const int lo = threadIdx.x * per;
  const int hi = min(n, lo + per);
  uint32_t c_gt = 0, c_eq = 0;
  for (int i = lo; i < hi; ++i) {
    const uint32_t u = get(i);
    c_gt += u > T;
    c_eq += u == T;
  }
  int p_gt = static_cast<int>(block_inclusive_scan(c_gt, tmp) - c_gt);
  int p_eq = n_gt + static_cast<int>(block_inclusive_scan(c_eq, tmp) - c_eq);
  for (int i = lo; i < hi; ++i) {
    const uint32_t u = get(i);
    if (u > T && p_gt < n_gt) {
      out_key[p_gt] = u;
      out_idx[p_gt] = idx_of(i);
      ++p_gt;
    } else if (u == T && p_eq < k) {
      out_key[p_eq] = u;
      out_idx[p_eq] = idx_of(i);
      ++p_eq;
    }
  }
  return k;
}

struct IndexerArgs {
  const float* q;        // [B, IH, IC] fp32
  const float* w;        // [B, IH] fp32
  const void* keys;      // fp32 [B,S,IC] or codes [B,S,IC|IC/2]
  const float* kscale;   // [B,S] (quantised keys)
  const float* diag;     // [IC] (quantised keys)
  const int32_t* valid;  // [B] or null
  int64_t S;
  int64_t T;             // rows per key row: row b scores the keys of key row b / T
  int IH, IC, k, mode, n_chunks;
  float wscale;          // fp32(IC ** -0.5) for the query rotation
  uint32_t* cand_key;    // [B, n_chunks, k]
  int32_t* cand_idx;     // [B, n_chunks, k]
  int32_t* cand_cnt;     // [B, n_chunks]
};

template <int FMT>
__global__ __launch_bounds__(kThreads) void idx_score_chunk_kernel(IndexerArgs a) {
  __shared__ float qs[kMaxIH * kMaxIC / 4];  // IH*IC <= 4096 floats
  __shared__ float qs2[FMT == kKeyF32 ? 1 : kMaxIH * kMaxIC / 4];
  __shared__ float wa[kMaxIH];
  __shared__ uint32_t sc[kChunk];
  __shared__ uint32_t hist[kThreads];
  __shared__ uint32_t tmp[kThreads];
  __shared__ uint32_t bcast[2];

  const int b = blockIdx.y;
  const int chunk = blockIdx.x;
  const int IH = a.IH, IC = a.IC;
  const int64_t S = a.S;
  const int64_t nv = a.valid ? min<int64_t>(S, max(0, a.valid[b])) : S;
  const int64_t j0 = static_cast<int64_t>(chunk) * kChunk;
  const int n = static_cast<int>(max<int64_t>(0, min<int64_t>(kChunk, nv - j0)));
  int32_t* cnt_out = a.cand_cnt + static_cast<int64_t>(b) * a.n_chunks + chunk;
  if (n <= 0) {
    if (threadIdx.x == 0) *cnt_out = 0;
    return;
  }

  // query (rotated for quantised keys) and head weights
  for (int i = threadIdx.x; i < IH * IC; i += kThreads) {
    float v = a.q[static_cast<int64_t>(b) * IH * IC + i];
    if constexpr (FMT != kKeyF32) v = v * a.diag[i % IC];
    qs[i] = v;
  }
  for (int h = threadIdx.x; h < IH; h += kThreads) {
    const float wv = a.w[static_cast<int64_t>(b) * IH + h];
    wa[h] = a.mode == AEKV_IDX_SOFTPLUS ? softplus_f32(wv) : (a.mode == AEKV_IDX_RELU_W ? fmaxf(wv, 0.0f) : wv);
  }
  __syncthreads();
  if constexpr (FMT != kKeyF32) {
    // q~ = _wht(diag * q) per head, ping-ponging between qs and qs2 (stage order h = 1, 2, ...).
    float* src = qs;
    float* dst = qs2;
    const int pairs = IH * IC / 2;
    for (int hh = 1; hh < IC; hh <<= 1) {
      for (int p = threadIdx.x; p < pairs; p += kThreads) {
        const int head = p / (IC / 2), r = p % (IC / 2);
        const int i = head * IC + (r / hh) * 2 * hh + (r % hh);
        const float x = src[i], y = src[i + hh];
        dst[i] = x + y;
        dst[i + hh] = x - y;
      }
      __syncthreads();
      float* t = src;
      src = dst;
      dst = t;
    }
    for (int i = threadIdx.x; i < IH * IC; i += kThreads) qs[i] = src[i] * a.wscale;
    __syncthreads();
  }

  // scores
  for (int t = threadIdx.x; t < n; t += kThreads) {
    const int64_t j = j0 + t;
    const int64_t row = static_cast<int64_t>(b) / a.T * S + j;
    float acc = 0.0f;
    for (int h = 0; h < IH; ++h) {
      const float* qh = qs + h * IC;
      float dot = 0.0f;
      if constexpr (FMT == kKeyF32) {
        const float* kp = static_cast<const float*>(a.keys) + row * IC;
        for (int c = 0; c < IC; ++c) dot = fmaf(qh[c], kp[c], dot);
      } else if constexpr (FMT == kKeyQ8) {
        const int8_t* kp = static_cast<const int8_t*>(a.keys) + row * IC;
        for (int c = 0; c < IC; ++c) dot = fmaf(qh[c], static_cast<float>(kp[c]), dot);
      } else {
        const uint8_t* kp = static_cast<const uint8_t*>(a.keys) + row * (IC / 2);
        for (int c = 0; c < IC / 2; ++c) {
          const uint32_t byte = kp[c];
          const int lo = (static_cast<int>(byte & 0x0fu) ^ 8) - 8;
          const int hi = (static_cast<int>(byte >> 4) ^ 8) - 8;
          dot = fmaf(qh[2 * c], static_cast<float>(lo), dot);
          dot = fmaf(qh[2 * c + 1], static_cast<float>(hi), dot);
        }
      }
      if (a.mode == AEKV_IDX_RELU_W) {
        acc = fmaf(wa[h], dot, acc);
      } else {
        acc = fmaf(wa[h], fmaxf(dot, 0.0f), acc);
      }
    }
    if constexpr (FMT != kKeyF32) acc = acc * a.kscale[row];
    sc[t] = order_key(acc);
  }
  __syncthreads();

  const int64_t cbase = (static_cast<int64_t>(b) * a.n_chunks + chunk) * a.k;
  const int cnt = select_compact([&](int i) { return sc[i]; }, [&](int i) { return static_cast<int32_t>(j0 + i); }, n,
                                 a.k, hist, tmp, bcast, a.cand_key + cbase, a.cand_idx + cbase);
  if (threadIdx.x == 0) *cnt_out = cnt;
}

__global__ __launch_bounds__(kThreads) void idx_merge_kernel(const uint32_t* __restrict__ cand_key,
                                                             const int32_t* __restrict__ cand_idx,
                                                             const int32_t* __restrict__ cand_cnt, int n_chunks, int k,
                                                             int64_t* __restrict__ out_idx,
                                                             float* __restrict__ out_score) {
  __shared__ uint64_t srt[kMaxK];
  __shared__ uint32_t sel_key[kMaxK];
  __shared__ int32_t sel_idx[kMaxK];
  __shared__ int32_t offs[kThreads + 1];
  __shared__ uint32_t hist[kThreads];
  __shared__ uint32_t tmp[kThreads];
  __shared__ uint32_t bcast[2];
  __shared__ int32_t chunk_start[1024 + 1];

  const int b = blockIdx.x;
  const uint32_t* ck = cand_key + static_cast<int64_t>(b) * n_chunks * k;
  const int32_t* ci = cand_idx + static_cast<int64_t>(b) * n_chunks * k;
  const int32_t* cc = cand_cnt + static_cast<int64_t>(b) * n_chunks;
  (void)offs;

  // prefix of chunk counts (n_chunks <= 1024 enforced on the host)
  if (threadIdx.x == 0) {
    int s = 0;
    for (int c = 0; c < n_chunks; ++c) {
      chunk_start[c] = s;
      s += cc[c];
    }
    chunk_start[n_chunks] = s;
  }
  __syncthreads();
  const int n = chunk_start[n_chunks];
  // candidate position -> (chunk, slot) lookup by binary search over chunk_start
  auto locate = [&](int i) -> int64_t {
    int lo = 0, hi = n_chunks - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (chunk_start[mid] <= i) lo = mid; else hi = mid - 1;
    }
    return static_cast<int64_t>(lo) * k + (i - chunk_start[lo]);
  };
  const int cnt = select_compact([&](int i) { return ck[locate(i)]; }, [&](int i) { return ci[locate(i)]; }, n, k, hist,
                                 tmp, bcast, sel_key, sel_idx);
  __syncthreads();

  // bitonic sort of (~key, idx) ascending == key desc, idx asc
  int P = 1;
  while (P < k) P <<= 1;
  for (int i = threadIdx.x; i < P; i += kThreads)
    srt[i] = i < cnt ? (static_cast<uint64_t>(~sel_key[i]) << 32) | static_cast<uint32_t>(sel_idx[i]) : ~0ull;
  __syncthreads();
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < P / 2; i += kThreads) {
        const int pos = 2 * i - (i & (stride - 1));
        const int partner = pos + stride;
        const bool up = (pos & size) == 0;
        const uint64_t x = srt[pos], y = srt[partner];
        if ((x > y) == up) {
          srt[pos] = y;
          srt[partner] = x;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < k; i += kThreads) {
    const bool ok = i < cnt;
    const uint64_t v = srt[i];
    out_idx[static_cast<int64_t>(b) * k + i] = ok ? static_cast<int64_t>(static_cast<uint32_t>(v & 0xffffffffu)) : -1;
    if (out_score)
      out_score[static_cast<int64_t>(b) * k + i] =
          ok ? order_key_inv(~static_cast<uint32_t>(v >> 32)) : -__builtin_inff();
  }
}

struct WsLayout {
  size_t key_off, idx_off, cnt_off, total;
};

WsLayout ws_layout(int64_t B, int64_t S, int32_t k) {
  const int64_t n_chunks = S > 0 ? ceil_div(S, kChunk) : 1;
  WsLayout l;
  const size_t nc = static_cast<size_t>(B * n_chunks * k);
  l.key_off = 0;
  l.idx_off = align_up(nc * 4, 256);
  l.cnt_off = l.idx_off + align_up(nc * 4, 256);
  l.total = l.cnt_off + align_up(static_cast<size_t>(B * n_chunks) * 4, 256);
  return l;
}

int validate_common(const float* q, const float* w, int64_t B, int64_t S, int32_t IH, int32_t IC, int32_t k,
                    int32_t mode, void* ws, size_t ws_bytes, int64_t* out_idx, const char* who) {
  if (B < 0 || S < 0) return fail(AEKV_ERR_SHAPE, "%s: negative B/S", who);
  if (IH < 1 || IH > kMaxIH) return fail(AEKV_ERR_UNSUPPORTED, "%s: IH=%d outside [1, %d]", who, IH, kMaxIH);
  if (IC < 1 || IC > kMaxIC || IH * IC > kMaxIH * kMaxIC / 4)
    return fail(AEKV_ERR_UNSUPPORTED, "%s: IC=%d (IH*IC=%d) outside the supported range (IC<=%d, IH*IC<=%d)", who, IC,
                IH * IC, kMaxIC, kMaxIH * kMaxIC / 4);
  if (k <= 0) return fail(AEKV_ERR_VALUE, "k must be positive");
  if (k > kMaxK) return fail(AEKV_ERR_UNSUPPORTED, "%s: k=%d exceeds the supported maximum %d", who, k, kMaxK);
  if (mode < 0 || mode > 2) return fail(AEKV_ERR_VALUE, "%s: unknown score mode %d", who, mode);
  if (S > static_cast<int64_t>(kChunk) * 1024)
    return fail(AEKV_ERR_UNSUPPORTED, "%s: S=%lld exceeds %d", who, (long long)S, kChunk * 1024);
  if (B > 65535) return fail(AEKV_ERR_UNSUPPORTED, "%s: B=%lld exceeds 65535", who, (long long)B);
  if (B > 0 && (!q || !w || !out_idx)) return fail(AEKV_ERR_VALUE, "%s: null pointer", who);
  const size_t need = std::max(ws_layout(B, S, k).total, mfma_indexer_workspace(B, S, k));
  if (B > 0 && (!ws || ws_bytes < need))
    return fail(AEKV_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who, need, ws_bytes);
  if (ws && !is_aligned(ws, 256)) return fail(AEKV_ERR_ALIGN, "%s: workspace must be 256-byte aligned", who);
  return AEKV_OK;
}

int launch_indexer(int fmt, IndexerArgs a, int64_t B, int64_t S, void* ws, int64_t* out_idx, float* out_score,
                   hipStream_t st, const char* who) {
  const WsLayout l = ws_layout(B, S, a.k);
  const int n_chunks = static_cast<int>(S > 0 ? ceil_div(S, kChunk) : 1);
  a.n_chunks = n_chunks;
  a.cand_key = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + l.key_off);
  a.cand_idx = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + l.idx_off);
  a.cand_cnt = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + l.cnt_off);
  a.S = S;
  a.wscale = wht_scale(a.IC);
  const dim3 g1(static_cast<uint32_t>(n_chunks), static_cast<uint32_t>(B));
  if (fmt == kKeyF32) hipLaunchKernelGGL(idx_score_chunk_kernel<kKeyF32>, g1, dim3(kThreads), 0, st, a);
  else if (fmt == kKeyQ8) hipLaunchKernelGGL(idx_score_chunk_kernel<kKeyQ8>, g1, dim3(kThreads), 0, st, a);
  else hipLaunchKernelGGL(idx_score_chunk_kernel<kKeyQ4>, g1, dim3(kThreads), 0, st, a);
  if (int rc = check_launch(who)) return rc;
  hipLaunchKernelGGL(idx_merge_kernel, dim3(static_cast<uint32_t>(B)), dim3(kThreads), 0, st, a.cand_key, a.cand_idx,
                     a.cand_cnt, n_chunks, a.k, out_idx, out_score);
  return check_launch(who);
}

}  // namespace
}  // namespace aekv

using namespace aekv;

extern "C" size_t aekv_csa_indexer_workspace_size(int64_t B, int64_t S, int32_t k) {
  if (B <= 0 || k <= 0) return 256;
  return std::max(ws_layout(B, S, k).total, mfma_indexer_workspace(B, S, k));
}

extern "C" int aekv_csa_indexer_topk(const float* index_q, const float* index_kv, const float* index_weight,
                                     const int32_t* valid, int64_t B, int64_t S, int32_t IH, int32_t IC, int32_t k,
                                     int32_t mode, void* ws, size_t ws_bytes, int64_t* out_idx, float* out_score,
                                     void* stream) {
  const char* who = "aekv_csa_indexer_topk";
  if (int rc = validate_common(index_q, index_weight, B, S, IH, IC, k, mode, ws, ws_bytes, out_idx, who)) return rc;
  if (B == 0) return AEKV_OK;
  if (S > 0 && !index_kv) return fail(AEKV_ERR_VALUE, "%s: null index_kv", who);
  IndexerArgs a{};
  a.q = index_q;
  a.w = index_weight;
  a.keys = index_kv;
  a.valid = valid;
  a.T = 1;
  a.IH = IH;
  a.IC = IC;
  a.k = k;
  a.mode = mode;
  return launch_indexer(kKeyF32, a, B, S, ws, out_idx, out_score, as_stream(stream), who);
}

// host-side checks of a quantised-key launch of B * T rows (no HIP call)
int aekv::validate_quant_rows(const float* index_q, const float* index_weight, const void* key_codes,
                        const float* key_scale, const float* diag, int64_t B, int64_t T, int64_t S, int32_t IH,
                        int32_t IC, int32_t bits, int32_t k, int32_t mode, void* ws, size_t ws_bytes,
                        int64_t* out_idx, const char* who) {
  if (bits != 4 && bits != 8) return fail(AEKV_ERR_VALUE, "bits must be 4 or 8, got %d", bits);
  if (!is_pow2(IC)) return fail(AEKV_ERR_VALUE, "WHT requires last dim to be a power of 2, got %d", IC);
  if (bits == 4 && IC < 2) return fail(AEKV_ERR_VALUE, "4-bit packing needs an even last dim, got %d", IC);
  if (B < 0 || T < 1) return fail(AEKV_ERR_SHAPE, "%s: B=%lld T=%lld", who, (long long)B, (long long)T);
  if (B > 0 && T > 65535 / B) return fail(AEKV_ERR_UNSUPPORTED, "%s: B*T exceeds 65535", who);
  const int64_t rows = B * T;
  if (int rc = validate_common(index_q, index_weight, rows, S, IH, IC, k, mode, ws, ws_bytes, out_idx, who)) return rc;
  if (rows > 0 && S > 0 && (!key_codes || !key_scale || !diag)) return fail(AEKV_ERR_VALUE, "%s: null key pointer", who);
  return AEKV_OK;
}

namespace {

// rows = B * T query rows; row r scores the codes of key row r / T
int topk_quant_rows(const float* index_q, const float* index_weight, const void* key_codes, const float* key_scale,
                    const float* diag, const int32_t* valid, int64_t B, int64_t T, int64_t S, int32_t IH, int32_t IC,
                    int32_t bits, int32_t k, int32_t mode, void* ws, size_t ws_bytes, int64_t* out_idx,
                    float* out_score, void* stream, const char* who) {
  if (int rc = validate_quant_rows(index_q, index_weight, key_codes, key_scale, diag, B, T, S, IH, IC, bits, k, mode,
                                   ws, ws_bytes, out_idx, who))
    return rc;
  const int64_t rows = B * T;
  if (rows == 0) return AEKV_OK;
  if (use_specialised_codec() && mfma_indexer_supported(IH, IC, k, S))
    return launch_mfma_indexer(index_q, index_weight, key_codes, key_scale, diag, valid, rows, T, S, IH, IC, bits, k,
                               mode, ws, out_idx, out_score, as_stream(stream), who);
  IndexerArgs a{};
  a.q = index_q;
  a.w = index_weight;
  a.keys = key_codes;
  a.kscale = key_scale;
  a.diag = diag;
  a.valid = valid;
  a.T = T;
  a.IH = IH;
  a.IC = IC;
  a.k = k;
  a.mode = mode;
  return launch_indexer(bits == 8 ? kKeyQ8 : kKeyQ4, a, rows, S, ws, out_idx, out_score, as_stream(stream), who);
}

}  // namespace

extern "C" int aekv_csa_indexer_topk_quant(const float* index_q, const float* index_weight, const void* key_codes,
                                           const float* key_scale, const float* diag, const int32_t* valid, int64_t B,
                                           int64_t S, int32_t IH, int32_t IC, int32_t bits, int32_t k, int32_t mode,
                                           void* ws, size_t ws_bytes, int64_t* out_idx, float* out_score,
                                           void* stream) {
  return topk_quant_rows(index_q, index_weight, key_codes, key_scale, diag, valid, B, 1, S, IH, IC, bits, k, mode, ws,
                         ws_bytes, out_idx, out_score, stream, "aekv_csa_indexer_topk_quant");
}

// ---- allocation-free variant --------------------------------------------------------------
// The workspace lives in a file-scope device array, one copy per GPU the library runs on, held
// until the process ends.  In host code `scratch` names a host-side stand-in, so its device address
// is looked up once per device (hipGetSymbolAddress with that device current) and only that
// address is ever handed to kernels.  The kernels write every workspace word they later read
// within the same call (order keys, slot maxima, per-chunk candidate counts), so nothing has to
// be cleared between calls; calls that overlap on one GPU share the array and race.
static __device__ __align__(256) unsigned char scratch[AEKV_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxScratchDevices] = {};

int static_scratch(hipStream_t st, void** addr, const char* who) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(AEKV_ERR_HIP, "%s: hipGetDevice failed", who);
  if (st) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(st, &sdev) != hipSuccess) return fail(AEKV_ERR_HIP, "%s: hipStreamGetDevice failed", who);
    if (sdev != dev)
      return fail(AEKV_ERR_VALUE, "%s: the stream belongs to device %d, the current device is %d", who,
                  static_cast<int>(sdev), dev);
  }
  if (dev < 0 || dev >= kMaxScratchDevices) return fail(AEKV_ERR_UNSUPPORTED, "%s: device %d out of range", who, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(AEKV_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: HIP error %d (%s)", who, dev,
                  static_cast<int>(e), hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return AEKV_OK;
}

}  // namespace

extern "C" int aekv_csa_indexer_topk_quant_noalloc(const float* index_q, const float* index_weight,
                                                   const void* key_codes, const float* key_scale, const float* diag,
                                                   const int32_t* valid, int64_t B, int64_t S, int32_t IH, int32_t IC,
                                                   int32_t bits, int32_t k, int32_t mode, int64_t* out_idx,
                                                   float* out_score, void* stream) {
  const char* who = "aekv_csa_indexer_topk_quant_noalloc";
  // the workspace entry point's argument checks first, with the workspace check deferred (no HIP call)
  void* const placeholder = reinterpret_cast<void*>(static_cast<uintptr_t>(256));
  if (int rc = validate_quant_rows(index_q, index_weight, key_codes, key_scale, diag, B, 1, S, IH, IC, bits, k, mode,
                                   placeholder, SIZE_MAX, out_idx, who))
    return rc;
  if (B == 0) return AEKV_OK;
  const size_t need = aekv_csa_indexer_workspace_size(B, S, k);
  if (need > AEKV_STATIC_SCRATCH_BYTES)
    return fail(AEKV_ERR_UNSUPPORTED,
                "%s: B=%lld S=%lld k=%d needs %zu bytes of scratch, more than the static %zu bytes; use "
                "aekv_csa_indexer_topk_quant with a caller workspace",
                who, static_cast<long long>(B), static_cast<long long>(S), k, need,
                static_cast<size_t>(AEKV_STATIC_SCRATCH_BYTES));
  void* ws = nullptr;
  if (int rc = static_scratch(as_stream(stream), &ws, who)) return rc;
  return topk_quant_rows(index_q, index_weight, key_codes, key_scale, diag, valid, B, 1, S, IH, IC, bits, k, mode, ws,
                         AEKV_STATIC_SCRATCH_BYTES, out_idx, out_score, stream, who);
}

extern "C" int aekv_csa_prefill_indexer_topk_quant(const float* index_q, const float* index_weight,
                                                   const void* key_codes, const float* key_scale, const float* diag,
                                                   const int32_t* valid, int64_t B, int64_t T, int64_t S, int32_t IH,
                                                   int32_t IC, int32_t bits, int32_t k, int32_t mode, void* ws,
                                                   size_t ws_bytes, int64_t* out_idx, float* out_score,
                                                   void* stream) {
  return topk_quant_rows(index_q, index_weight, key_codes, key_scale, diag, valid, B, T, S, IH, IC, bits, k, mode, ws,
                         ws_bytes, out_idx, out_score, stream, "aekv_csa_prefill_indexer_topk_quant");
}
