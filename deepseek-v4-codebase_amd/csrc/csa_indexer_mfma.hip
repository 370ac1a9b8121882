// CSA lightning indexer over TurboQuant-coded index keys on the gfx950 matrix cores, with an
// exact top-k that needs no atomics.
//
// Reference: aether_2b/modeling.py:604-616 and aether_2b/serving.py:606-621 (score rules, top-k);
// the keys are PolarQuant codes (turbo_quant.py:127-211).
//
// Scoring.  q.k_j = scale_j * (q~ . codes_j) with q~ = WHT(diag * q) (the WHT is orthogonal and
// symmetric).  Per head, q~ is split into four int8 digits with a common power-of-two step S_h:
//   q~ = S_h * (d0 + 2^-7 d1 + 2^-14 d2 + 2^-21 d3) + r,   |d_i| <= 64,   |r| <= S_h * 2^-22,
// and v_mfma_i32_16x16x64_i8 computes the exact integer dots I_i = d_i . codes_j for 16 keys at a
// time (A rows = 4 heads x 4 digits; B columns = keys; 4-bit codes enter as 16*code, the nibble
// shifted to the top of its byte).  The 16x16 result leaves each lane with the four digit dots of
// one (head, key); they are combined in fp32 with the head weight folded in, clamped (relu), summed
// over heads across lane groups and multiplied by scale_j.  The only approximation is r (relative
// ~2^-27 of max|q~_h|) and three fp32 roundings, i.e. fp32-level scores.
//
// Selection.  A wave owns 2048 consecutive keys, 32 per lane (slot s, lane l <-> key base+64s+l),
// as order-preserving uint32 keys (invalid keys = 0, below every finite score).  The k-th largest
// key T is found by a 32-step binary search whose counts are ballot popcounts; the wave then
// compacts keys > T and the first (k - #>T) keys == T in index order (ballot + mbcnt), which is the
// top-k under (score desc, index asc).  A merge kernel repeats this over the candidates of a row
// (in rounds of 2048 carrying the current best k), and sorts the final k.  Because the order is
// total, every element of the row's top-k is in its wave's top-k, so the result is exact.
#include "aekv_common.h"

namespace aekv {
namespace {

constexpr int kThreads = 256;
constexpr int kSlots = 32;                    // keys per lane in a wave's selection window
constexpr int kWaveKeys = 64 * kSlots;        // 2048
constexpr int kChunkKeys = 4 * kWaveKeys;     // keys per workgroup
constexpr int kMaxMfmaK = 1024;
constexpr int kMaxLists = 2048;               // wave chunks per row (S <= 4M keys)

typedef __attribute__((ext_vector_type(4))) int i32x4_t;

__device__ __forceinline__ float softplus_f32(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

__device__ __forceinline__ int mbcnt64(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
}

__device__ __forceinline__ int popc64(uint64_t m) { return __builtin_popcountll(m); }

// k-th largest (k >= 1) of the wave's 64*SLOTS keys (binary search on the value, 32 steps).
template <int SLOTS>
__device__ __forceinline__ uint32_t wave_kth(const uint32_t (&key)[SLOTS], int k) {
  uint32_t T = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t tc = T | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) cnt += popc64(__builtin_amdgcn_ballot_w64(key[s] >= tc));
    if (cnt >= k) T = tc;
  }
  return T;
}

// Writes the top-k (k <= #keys > 0) of the wave's keys in index order of (slot, lane), first those
// > T then those == T; idx(s) gives the lane's element index for slot s.  Returns the count.
template <int SLOTS, typename IdxFn>
__device__ __forceinline__ int wave_compact(const uint32_t (&key)[SLOTS], uint32_t T, int k, IdxFn idx,
                                            uint32_t* out_key, int32_t* out_idx) {
  int n_gt = 0;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) n_gt += popc64(__builtin_amdgcn_ballot_w64(key[s] > T));
  int pos_gt = 0, pos_eq = n_gt;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const uint64_t m_gt = __builtin_amdgcn_ballot_w64(key[s] > T);
    const uint64_t m_eq = __builtin_amdgcn_ballot_w64(key[s] == T);
    if (key[s] > T) {
      const int p = pos_gt + mbcnt64(m_gt);
      out_key[p] = key[s];
      out_idx[p] = idx(s);
    } else if (key[s] == T) {
      const int p = pos_eq + mbcnt64(m_eq);
      if (p < k) {
        out_key[p] = key[s];
        out_idx[p] = idx(s);
      }
    }
    pos_gt += popc64(m_gt);
    pos_eq += popc64(m_eq);
  }
  return k;
}

// Top-k of the wave's keys, keys equal to 0 never selected.  Returns the count written.
template <int SLOTS, typename IdxFn>
__device__ __forceinline__ int wave_topk(const uint32_t (&key)[SLOTS], int k, IdxFn idx, uint32_t* out_key,
                                         int32_t* out_idx) {
  int n_valid = 0;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) n_valid += popc64(__builtin_amdgcn_ballot_w64(key[s] != 0u));
  const int kk = min(k, n_valid);
  if (kk == 0) return 0;
  const uint32_t T = wave_kth<SLOTS>(key, kk);
  return wave_compact<SLOTS>(key, T, kk, idx, out_key, out_idx);
}

struct MfmaIdxArgs {
  const float* q;        // [B, IH, IC]
  const float* w;        // [B, IH]
  const uint8_t* codes;  // [B, S, IC or IC/2]
  const float* kscale;   // [B, S]
  const float* diag;     // [IC]
  const int32_t* valid;  // [B] or null
  int64_t S;
  int IH, k, mode, n_wchunks;  // n_wchunks: 2048-key wave chunks per row
  float wscale;
  uint32_t* cand_key;    // [B, n_wchunks, k]
  int32_t* cand_idx;     // [B, n_wchunks, k]
  int32_t* cand_cnt;     // [B, n_wchunks]
};

// digit position -> index c of the key element for lane group g, byte position p of k-step ks
template <int BITS>
__device__ __forceinline__ int cmap(int ks, int g, int p) {
  if constexpr (BITS == 8) {
    return 64 * ks + 16 * g + p;
  } else {
    // the lane loads bytes 8g..8g+7 of the 32-byte k-step: dwords (lo nibbles of bytes 0-3,
    // hi nibbles of bytes 0-3, lo of 4-7, hi of 4-7)
    const int q4 = p >> 2, r = p & 3;
    return 64 * ks + 16 * g + 8 * (q4 >> 1) + 2 * r + (q4 & 1);
  }
}

template <int BITS, int IC, int NRB>
__global__ __launch_bounds__(kThreads) void idx_mfma_score_kernel(MfmaIdxArgs a) {
  constexpr int KS = IC / 64;          // k-steps of 64
  constexpr int RB = BITS == 8 ? IC : IC / 2;
  __shared__ float qs[16 * IC];
  __shared__ float qs2[16 * IC];
  __shared__ int8_t dig[4][16][IC];
  __shared__ float hf[16][4];          // per head: digit factors S * 2^-7d (/16 for 4-bit) * weight
  __shared__ float hb[16][2];          // per head: clamp bounds
  // per wave: candidate keys [0, kMaxMfmaK) and indices [kMaxMfmaK, 2 kMaxMfmaK); the whole
  // 2048-word row also stages the slot keys before the selection
  __shared__ uint32_t wbuf[4][2 * kMaxMfmaK];
  static_assert(2 * kMaxMfmaK == kWaveKeys, "slot staging must fill exactly one wave buffer");

  const int b = blockIdx.y;
  const int IH = a.IH;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, g = lane >> 4;
  const int64_t S = a.S;
  const int64_t nv = a.valid ? min<int64_t>(S, max(0, a.valid[b])) : S;

  // ---- query rotation and digits (once per workgroup) ----
  for (int i = threadIdx.x; i < 16 * IC; i += kThreads) {
    const int h = i / IC, c = i % IC;
    qs[i] = h < IH ? a.q[(static_cast<int64_t>(b) * IH + h) * IC + c] * a.diag[c] : 0.0f;
  }
  __syncthreads();
  {
    float* src = qs;
    float* dst = qs2;
    for (int hh = 1; hh < IC; hh <<= 1) {
      for (int p = threadIdx.x; p < 16 * IC / 2; p += kThreads) {
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
    if (src != qs)
      for (int i = threadIdx.x; i < 16 * IC; i += kThreads) qs[i] = src[i];
    __syncthreads();
  }
  if (wv == 0) {
    // one wave: per head, step S_h = 2^(e-6) from max|q~_h| = m * 2^e (m in [0.5, 1))
    for (int h = 0; h < 16; ++h) {
      float mx = 0.0f;
      for (int c = lane; c < IC; c += 64) mx = fmaxf(mx, fabsf(qs[h * IC + c] * a.wscale));
      mx = wave_max(mx);
      int e = 0;
      (void)frexpf(mx, &e);
      const float step = mx > 0.0f ? ldexpf(1.0f, e - 6) : 1.0f;
      for (int c = lane; c < IC; c += 64) {
        float r = qs[h * IC + c] * a.wscale;  // q~ = _wht(diag * q)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float sd = ldexpf(step, -7 * d);
          const float di = rintf(r / sd);  // exact quotient by a power of two
          r = fmaf(-di, sd, r);            // exact residual
          dig[d][h][c] = static_cast<int8_t>(di);
        }
      }
      if (lane == 0) {
        float wa = 0.0f, lo = -__builtin_inff(), hi = __builtin_inff();
        if (h < IH) {
          const float wr = a.w[static_cast<int64_t>(b) * IH + h];
          if (a.mode == AEKV_IDX_SOFTPLUS) {
            wa = softplus_f32(wr);
            lo = 0.0f;
          } else if (a.mode == AEKV_IDX_RAW) {
            wa = wr;
            if (wr >= 0.0f) lo = 0.0f; else hi = 0.0f;  // relu(dot)*w = clamp(dot*w) toward 0
          } else {
            wa = fmaxf(wr, 0.0f);                       // relu on the weight only
          }
        }
        const float unit = BITS == 4 ? 1.0f / 16.0f : 1.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) hf[h][d] = ldexpf(step, -7 * d) * unit * wa;
        hb[h][0] = lo;
        hb[h][1] = hi;
      }
    }
  }
  __syncthreads();

  // A operands (digits) and combine constants for this lane
  i32x4_t A[NRB][KS];
  float f[NRB][4], lo[NRB], hi[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int row = lane & 15;
    const int h = 4 * rb + (row >> 2), d = row & 3;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int dw = 0; dw < 4; ++dw) {
        uint32_t word = 0;
#pragma unroll
        for (int by = 0; by < 4; ++by) {
          const int c = cmap<BITS>(ks, g, 4 * dw + by);
          word |= (static_cast<uint32_t>(static_cast<uint8_t>(dig[d][h][c])) << (8 * by));
        }
        A[rb][ks][dw] = static_cast<int>(word);
      }
    }
    const int ho = 4 * rb + g;  // output rows 4g..4g+3 = head 4rb+g, digits 0..3
#pragma unroll
    for (int d2 = 0; d2 < 4; ++d2) f[rb][d2] = hf[ho][d2];
    lo[rb] = hb[ho][0];
    hi[rb] = hb[ho][1];
  }

  // ---- scoring: this wave's 2048 keys ----
  const int64_t kb = static_cast<int64_t>(blockIdx.x) * kChunkKeys + static_cast<int64_t>(wv) * kWaveKeys;
  const uint8_t* crow = a.codes + static_cast<int64_t>(b) * S * RB;
  const float* srow = a.kscale + static_cast<int64_t>(b) * S;
  // slot keys are staged in this wave's candidate buffer (ck/ci as one 2048-word array) and read
  // back into registers before the selection overwrites it
  uint32_t* sk = &wbuf[wv][0];
  uint32_t* ck = &wbuf[wv][0];
  int32_t* ci = reinterpret_cast<int32_t*>(&wbuf[wv][kMaxMfmaK]);
#pragma unroll 1
  for (int s = 0; s < kSlots; ++s) {
    uint32_t kq[4];
#pragma unroll
    for (int tq = 0; tq < 4; ++tq) {
      const int64_t j = kb + 64 * s + 16 * tq + (lane & 15);
      const bool okj = j < nv;
      const int64_t jr = okj ? j : 0;
      i32x4_t acc[NRB];
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) acc[rb] = i32x4_t{0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        i32x4_t B;
        if constexpr (BITS == 8) {
          const uint4 v = okj ? *reinterpret_cast<const uint4*>(crow + jr * RB + 64 * ks + 16 * g) : make_uint4(0, 0, 0, 0);
          B = i32x4_t{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
        } else {
          const uint2 v = okj ? *reinterpret_cast<const uint2*>(crow + jr * RB + 32 * ks + 8 * g) : make_uint2(0, 0);
          B = i32x4_t{static_cast<int>((v.x << 4) & 0xF0F0F0F0u), static_cast<int>(v.x & 0xF0F0F0F0u),
                      static_cast<int>((v.y << 4) & 0xF0F0F0F0u), static_cast<int>(v.y & 0xF0F0F0F0u)};
        }
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) acc[rb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[rb][ks], B, acc[rb], 0, 0, 0);
      }
      float t = 0.0f;
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        float v = static_cast<float>(acc[rb][0]) * f[rb][0];
        v = fmaf(static_cast<float>(acc[rb][1]), f[rb][1], v);
        v = fmaf(static_cast<float>(acc[rb][2]), f[rb][2], v);
        v = fmaf(static_cast<float>(acc[rb][3]), f[rb][3], v);
        t += __builtin_amdgcn_fmed3f(v, lo[rb], hi[rb]);
      }
      t += xor_lane<16>(t);  // sum over the four head groups
      t += xor_lane<32>(t);
      const float sc = t * srow[jr];
      kq[tq] = okj ? order_key(sc) : 0u;
    }
    const uint32_t mine = g == 0 ? kq[0] : (g == 1 ? kq[1] : (g == 2 ? kq[2] : kq[3]));
    sk[64 * s + lane] = mine;  // slot s of lane l at 64s + l
  }
  __builtin_amdgcn_wave_barrier();
  uint32_t key[kSlots];
#pragma unroll
  for (int s = 0; s < kSlots; ++s) key[s] = sk[64 * s + lane];
  __builtin_amdgcn_wave_barrier();

  // ---- per-wave exact top-k ----
  const int cnt = wave_topk<kSlots>(key, a.k, [&](int s) { return static_cast<int32_t>(kb + 64 * s + lane); }, ck, ci);
  __builtin_amdgcn_wave_barrier();
  const int64_t wchunk = static_cast<int64_t>(blockIdx.x) * 4 + wv;
  if (wchunk < a.n_wchunks) {
    const int64_t base = (static_cast<int64_t>(b) * a.n_wchunks + wchunk) * a.k;
    for (int i = lane; i < cnt; i += 64) {
      a.cand_key[base + i] = ck[i];
      a.cand_idx[base + i] = ci[i];
    }
    if (lane == 0) a.cand_cnt[static_cast<int64_t>(b) * a.n_wchunks + wchunk] = cnt;
  }
}

// Merges the candidates get(e), e in [0, n), into the wave's held best (hk/hi, `held` entries) in
// rounds: the slots hold the current best followed by as many new candidates as fit.  Candidate
// order is index order for equal keys, so the result is the top-k under (key desc, index asc).
// Needs k <= kMaxMfmaK (< kWaveKeys) so every round consumes new candidates.
template <typename Get>
__device__ int wave_merge_rounds(int held, int n, int k, Get get, uint32_t* hk, int32_t* hi, uint32_t* stk,
                                 int32_t* sti) {
  const int lane = threadIdx.x & 63;
  int pos = 0;
  while (pos < n) {
    const int take = min(n - pos, kWaveKeys - held);
    // stage the round in LDS: [0, held) current best, [held, held + take) new, rest empty
#pragma unroll 1
    for (int e = lane; e < kWaveKeys; e += 64) {
      uint32_t kv = 0u;
      int32_t iv = 0;
      if (e < held) {
        kv = hk[e];
        iv = hi[e];
      } else if (e < held + take) {
        get(pos + e - held, kv, iv);
      }
      stk[e] = kv;
      sti[e] = iv;
    }
    __builtin_amdgcn_wave_barrier();
    uint32_t key[kSlots];
    int32_t idx[kSlots];
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      key[s] = stk[64 * s + lane];
      idx[s] = sti[64 * s + lane];
    }
    __builtin_amdgcn_wave_barrier();  // every lane has read the round before hk/hi are overwritten
    held = wave_topk<kSlots>(key, k, [&](int s) { return idx[s]; }, hk, hi);
    __builtin_amdgcn_wave_barrier();
    pos += take;
  }
  return held;
}

// Row merge: top-k of the row's candidates (n_wchunks lists of <= k each) -> sorted int64 indices.
__global__ __launch_bounds__(kThreads) void idx_mfma_merge_kernel(const uint32_t* __restrict__ cand_key,
                                                                  const int32_t* __restrict__ cand_idx,
                                                                  const int32_t* __restrict__ cand_cnt, int n_wchunks,
                                                                  int k, int64_t* __restrict__ out_idx,
                                                                  float* __restrict__ out_score) {
  __shared__ uint32_t hk[4][kMaxMfmaK];
  __shared__ int32_t hi[4][kMaxMfmaK];
  __shared__ uint32_t fk[kMaxMfmaK];
  __shared__ int32_t fi[kMaxMfmaK];
  __shared__ int held_w[4];
  __shared__ int pref[kMaxLists + 1];
  __shared__ uint64_t srt[kMaxMfmaK];
  __shared__ uint32_t stk[4][kWaveKeys];
  __shared__ int32_t sti[4][kWaveKeys];
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t* ckr = cand_key + static_cast<int64_t>(b) * n_wchunks * k;
  const int32_t* cir = cand_idx + static_cast<int64_t>(b) * n_wchunks * k;
  const int32_t* ccr = cand_cnt + static_cast<int64_t>(b) * n_wchunks;

  // prefix of list counts (exclusive), computed by one wave in blocks of 64
  if (wv == 0) {
    int run = 0;
    for (int l0 = 0; l0 < n_wchunks; l0 += 64) {
      const int l = l0 + lane;
      const int c = l < n_wchunks ? ccr[l] : 0;
      int incl = c;
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
      }
      if (l < n_wchunks) pref[l] = run + incl - c;
      run += __shfl(incl, 63, 64);
    }
    if (lane == 0) pref[n_wchunks] = run;
  }
  __syncthreads();

  // stage 1: wave wv reduces lists [l_lo, l_hi) to its best k
  const int per = (n_wchunks + 3) / 4;
  const int l_lo = min(n_wchunks, wv * per), l_hi = min(n_wchunks, l_lo + per);
  const int p_lo = pref[l_lo], p_hi = pref[l_hi];
  auto get1 = [&](int e, uint32_t& key, int32_t& idx) {
    const int P = p_lo + e;
    int lo = l_lo, hi2 = l_hi - 1;  // last list with pref <= P
    while (lo < hi2) {
      const int mid = (lo + hi2 + 1) >> 1;
      if (pref[mid] <= P) lo = mid; else hi2 = mid - 1;
    }
    const int64_t src = static_cast<int64_t>(lo) * k + (P - pref[lo]);
    key = ckr[src];
    idx = cir[src];
  };
  const int h1 = wave_merge_rounds(0, p_hi - p_lo, k, get1, hk[wv], hi[wv], stk[wv], sti[wv]);
  if (lane == 0) held_w[wv] = h1;
  __syncthreads();

  // stage 2: wave 0 merges the four lists (in wave order = index order)
  if (wv == 0) {
    const int c0 = held_w[0], c1 = held_w[1], c2 = held_w[2], c3 = held_w[3];
    auto get2 = [&](int e, uint32_t& key, int32_t& idx) {
      int w = 0, off = e;
      if (off >= c0) { off -= c0; w = 1;
        if (off >= c1) { off -= c1; w = 2;
          if (off >= c2) { off -= c2; w = 3; } } }
      key = hk[w][off];
      idx = hi[w][off];
    };
    const int h2 = wave_merge_rounds(0, c0 + c1 + c2 + c3, k, get2, fk, fi, stk[0], sti[0]);
    if (lane == 0) held_w[0] = h2;
  }
  __syncthreads();
  const int cnt = held_w[0];

  // bitonic sort of (~key, idx) ascending == key desc, idx asc
  int P = 1;
  while (P < k) P <<= 1;
  for (int i = threadIdx.x; i < P; i += kThreads)
    srt[i] = i < cnt ? (static_cast<uint64_t>(~fk[i]) << 32) | static_cast<uint32_t>(fi[i]) : ~0ull;
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

typedef void (*score_fn)(MfmaIdxArgs);

template <int BITS, int IC>
score_fn pick_nrb(int nrb) {
  switch (nrb) {
    case 1: return idx_mfma_score_kernel<BITS, IC, 1>;
    case 2: return idx_mfma_score_kernel<BITS, IC, 2>;
    case 3: return idx_mfma_score_kernel<BITS, IC, 3>;
    case 4: return idx_mfma_score_kernel<BITS, IC, 4>;
    default: return nullptr;
  }
}

}  // namespace

size_t mfma_indexer_workspace(int64_t B, int64_t S, int32_t k) {
  const int64_t n_wchunks = S > 0 ? ceil_div(S, kWaveKeys) : 1;
  const size_t nc = static_cast<size_t>(B * n_wchunks * k);
  return align_up(nc * 4, 256) * 2 + align_up(static_cast<size_t>(B * n_wchunks) * 4, 256);
}

bool mfma_indexer_supported(int IH, int IC, int k, int64_t S) {
  // S >= 1: the score loop reads the scale of key 0 for out-of-range lanes.
  return IH >= 1 && IH <= 16 && (IC == 64 || IC == 128) && k <= kMaxMfmaK && S >= 1 &&
         S <= static_cast<int64_t>(kMaxLists) * kWaveKeys;
}

int launch_mfma_indexer(const float* q, const float* w, const void* codes, const float* kscale, const float* diag,
                        const int32_t* valid, int64_t B, int64_t S, int IH, int IC, int bits, int k, int mode, void* ws,
                        int64_t* out_idx, float* out_score, hipStream_t st, const char* who) {
  MfmaIdxArgs a{};
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
  a.n_wchunks = static_cast<int>(S > 0 ? ceil_div(S, kWaveKeys) : 1);
  a.wscale = wht_scale(IC);
  const size_t nc = static_cast<size_t>(B * a.n_wchunks * k);
  a.cand_key = static_cast<uint32_t*>(ws);
  a.cand_idx = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + align_up(nc * 4, 256));
  a.cand_cnt = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + 2 * align_up(nc * 4, 256));
  const int nrb = (IH + 3) / 4;
  score_fn fn = nullptr;
  if (bits == 8) fn = IC == 64 ? pick_nrb<8, 64>(nrb) : pick_nrb<8, 128>(nrb);
  else fn = IC == 64 ? pick_nrb<4, 64>(nrb) : pick_nrb<4, 128>(nrb);
  if (!fn) return fail(AEKV_ERR_UNSUPPORTED, "%s: no matrix-core indexer for IH=%d IC=%d", who, IH, IC);
  const int n_wg = static_cast<int>(S > 0 ? ceil_div(S, kChunkKeys) : 1);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(n_wg), static_cast<uint32_t>(B)), dim3(kThreads), 0, st, a);
  if (int rc = check_launch(who)) return rc;
  hipLaunchKernelGGL(idx_mfma_merge_kernel, dim3(static_cast<uint32_t>(B)), dim3(kThreads), 0, st, a.cand_key,
                     a.cand_idx, a.cand_cnt, a.n_wchunks, k, out_idx, out_score);
  return check_launch(who);
}

}  // namespace aekv
