// CSA lightning indexer over TurboQuant-coded index keys on the gfx950 matrix cores, with an
// exact radix top-k.
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
// one (head, key); the digit pairs are joined exactly in int32 (|I_i| <= 64 * 128 * 128 = 2^20, so
// 2^7 I_0 + I_1 and 2^7 I_2 + I_3 stay below 2^28), converted and combined in fp32 with the head
// weight folded in, clamped (relu), summed over heads across lane groups and multiplied by
// scale_j.  The only approximation is r (relative ~2^-27 of max|q~_h|) and at most four fp32
// roundings, i.e. fp32-level scores.
//
// Kernels (one stream, in order):
//   score  (wide grid)  rotates the row's query and splits the digits in LDS (per workgroup),
//          scores every visible key, stores its order-preserving uint32 key and the max of every
//          16-key slot.
//   final  (one workgroup per row)  bounds the k-th largest key from below by the k-th largest
//          slot max (a histogram of the slot maxima in 1/128-binade bins below the row's largest),
//          reads only the slots that can hold a top-k key and keeps their keys above the bound.
//          Up to 1024 candidates (the usual case: a few hundred) are sorted outright, 64 per wave
//          in registers, the runs placed by binary search; more go through three LDS radix levels
//          (keys > T and the lowest-index keys == T, placed by rank under (key desc, index asc)).
//          If the candidates overflow LDS (many equal keys), the levels run over all of the row's
//          stored keys, read in index order.
// Both routes return the top-k under the total order (score desc, index asc).
//
// The select body (select_row) is shared by the select kernel and the fused CSA decode kernel,
// which continues with the row's attention in the same workgroup.
#pragma once

#include <type_traits>

#include <algorithm>

#include "aekv_common.h"

namespace aekv {
namespace idx {

constexpr int kThreads = 256;
constexpr int kSelThreads = 1024;
constexpr int kHistBins = 4096;      // slot-max histogram bins (key >> 16 below the row maximum)
constexpr int kCandCap = 4096;       // candidates a row's workgroup collects in LDS (fast route)
constexpr int kMaxMfmaK = 1024;
constexpr int kMaxNrb = 4;           // row blocks of 4 heads (IH <= 16)
constexpr int64_t kMaxKeys = int64_t(1) << 24;  // byte offsets within a key row fit in 32 bits (2^24 x 128)
constexpr int kScoreTT = 4;          // prefill rows sharing each key group in the score kernel
constexpr int64_t kScoreTargetWG = 2048;  // score workgroups the launch aims for

// Slots of 64 keys per score group (one group's codes per wave in registers): 256 keys of up to
// 32 code bytes, 128 of 64, 64 of 128.  Decode rows (TT = 1) keep two groups in flight, of half
// that size, so that the registers stay within eight waves per SIMD.
__host__ __device__ constexpr int score_spw(int bits, int ic, int tt) {
  const int rb = bits == 8 ? ic : ic / 2;
  const int spw = rb <= 32 ? 4 : (rb <= 64 ? 2 : 1);
  return tt == 1 && spw > 1 ? spw / 2 : spw;
}

typedef __attribute__((ext_vector_type(4))) int i32x4_t;

__device__ __forceinline__ float softplus_f32(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

__device__ __forceinline__ int mbcnt64(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
}

// Reserves v (< 2^NB) slots per active lane from the LDS counter *cnt with one atomic per wave
// (per-lane atomics on one LDS address serialise) and returns the lane's first slot.  The
// exclusive prefix sum over the active lanes comes from NB ballots.
template <int NB>
__device__ __forceinline__ uint32_t wave_reserve(uint32_t* cnt, uint32_t v) {
  uint32_t pre = 0u, tot = 0u;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const uint64_t m = __builtin_amdgcn_ballot_w64(((v >> b) & 1u) != 0u);
    pre += static_cast<uint32_t>(mbcnt64(m)) << b;
    tot += static_cast<uint32_t>(__builtin_popcountll(m)) << b;
  }
  uint32_t base = 0u;
  if (mbcnt64(__builtin_amdgcn_ballot_w64(true)) == 0 && tot != 0u) base = atomicAdd(cnt, tot);
  return __builtin_amdgcn_readfirstlane(base) + pre;
}

struct MfmaIdxArgs {
  const float* q;        // [B, IH, IC]
  const float* w;        // [B, IH]
  const uint8_t* codes;  // [B, S, IC or IC/2]
  const float* kscale;   // [B, S]
  const float* diag;     // [IC]
  const int32_t* valid;  // [B] or null
  int64_t S;
  int64_t T;             // rows per key row: row b scores the keys of key row b / T
  int IH, k, mode;
  int gpw;               // slot groups per wave in the score kernel
  float wscale;
  uint32_t* keys;        // [B][ks]                   order keys of visible keys
  int64_t ks;            // key row stride: S rounded up to a multiple of 16 (whole slots)
  uint32_t* smax;        // [B][ms]                   max order key of each 16-key slot
  int64_t ms;            // slot-max row stride: ceil(S / 16) rounded up to a multiple of 4
};

struct WsLayout {
  size_t keys, smax, total;
};

inline WsLayout layout(int64_t B, int64_t S) {
  WsLayout l{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align_up(bytes, 256);
    return at;
  };
  l.keys = take(static_cast<size_t>(B) * static_cast<size_t>(align_up(static_cast<size_t>(S), 16)) * 4);
  l.smax = take(static_cast<size_t>(B) * align_up((static_cast<size_t>(S) + 15) / 16, 4) * 4);
  l.total = o;
  return l;
}

// Counts read in place of a row's when a target lies past T (none) or a launch has no counts (all).
__device__ const int32_t kCountNone = 0;
__device__ const int32_t kCountAll = 0x7fffffff;

// Row b's visible count (b uniform over the workgroup; S without counts).  The count is read
// through the constant address space, which makes it a scalar load: the wait for it (where the
// null check's branch joins) leaves the vector memory counter alone, so it does not wait for
// vector requests issued before it (a vector load here had made that wait cover the caller's
// whole first memory round).  Integer compares: min<int64_t> lowers through doubles here.
__device__ __forceinline__ int64_t visible(const MfmaIdxArgs& a, int b) {
  if (!a.valid) return a.S;
  const int32_t v = *(const __attribute__((address_space(4))) int32_t*)(a.valid + b);
  return v <= 0 ? 0 : (v < a.S ? v : a.S);
}

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

// Sum over the four 16-lane groups ("rows") of t[q], delivered to row q: a reduce-scatter with
// three permlane swaps.  permlane16_swap(a, b) exchanges the odd rows of a with the even rows of b,
// so a' + b' holds a's pair sums (rows 0+1, 2+3) in rows 0 and 2 and b's in rows 1 and 3;
// permlane32_swap(u, w) exchanges u's upper half with w's lower half, so u' + w' holds u's half
// sums in rows 0-1 and w's in rows 2-3.  Every row ends with (t[q]_0 + t[q]_1) + (t[q]_2 + t[q]_3)
// for q = its row: the pairing of a butterfly sum, so the same fp32 value.  (The swap results are
// copied to scalars before the bit casts: hipcc lowers __builtin_bit_cast of element 1 of the
// builtin's result vector as element 0.)
__device__ __forceinline__ float row_sums_scatter(const float (&t)[4]) {
  auto sw16 = [](float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                    false, false);
    const uint32_t x0 = r[0], x1 = r[1];
    return __builtin_bit_cast(float, x0) + __builtin_bit_cast(float, x1);
  };
  const float u = sw16(t[0], t[1]), w = sw16(t[2], t[3]);
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, u), __builtin_bit_cast(uint32_t, w),
                                                  false, false);
  const uint32_t x0 = r[0], x1 = r[1];
  return __builtin_bit_cast(float, x0) + __builtin_bit_cast(float, x1);
}

template <int HL>
__device__ __forceinline__ uint32_t max_xor_u32(uint32_t v) {
  const uint32_t o = __builtin_bit_cast(uint32_t, xor_lane<HL>(__builtin_bit_cast(float, v)));
  return v > o ? v : o;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max_xor_u32<1>(v);
  v = max_xor_u32<2>(v);
  v = max_xor_u32<4>(v);
  v = max_xor_u32<8>(v);
  v = max_xor_u32<16>(v);
  return max_xor_u32<32>(v);
}

// 64-bit lane exchange with partner lane ^ j (j a power of two below 64, constant after unrolling).
__device__ __forceinline__ uint64_t xor_lane_u64(uint64_t v, int j) {
  float lo = __builtin_bit_cast(float, static_cast<uint32_t>(v));
  float hi = __builtin_bit_cast(float, static_cast<uint32_t>(v >> 32));
  switch (j) {
    case 1: lo = xor_lane<1>(lo); hi = xor_lane<1>(hi); break;
    case 2: lo = xor_lane<2>(lo); hi = xor_lane<2>(hi); break;
    case 4: lo = xor_lane<4>(lo); hi = xor_lane<4>(hi); break;
    case 8: lo = xor_lane<8>(lo); hi = xor_lane<8>(hi); break;
    case 16: lo = xor_lane<16>(lo); hi = xor_lane<16>(hi); break;
    default: lo = xor_lane<32>(lo); hi = xor_lane<32>(hi); break;
  }
  return (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, hi)) << 32) | __builtin_bit_cast(uint32_t, lo);
}

// Threshold search over a histogram: the largest bin t with sum_{u >= t} h[u] >= need, and
// above = sum_{u > t} h[u] (1 <= need <= sum of all bins).  Thread `tid` of NT owns the PER
// contiguous bins [PER*tid, PER*tid + PER), loaded as 16-byte vectors (global or LDS).
template <int PER>
__device__ __forceinline__ void load_bins(const uint32_t* h, int tid, uint32_t (&v)[PER]) {
  static_assert(PER % 4 == 0, "bins are loaded 4 at a time");
  const uint4* p = reinterpret_cast<const uint4*>(h + PER * tid);
#pragma unroll
  for (int i = 0; i < PER / 4; ++i) {
    const uint4 x = p[i];
    v[4 * i] = x.x;
    v[4 * i + 1] = x.y;
    v[4 * i + 2] = x.z;
    v[4 * i + 3] = x.w;
  }
}

// DPP move of x (lanes without a source, or in rows outside RMASK, read 0).
template <int CTRL, int RMASK = 0xF>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, RMASK, 0xF, true));
}

// Inclusive suffix sum over the lanes of a wave (lane 63 holds the highest bins): the inclusive
// prefix sum by DPP (row_shr 1, 2, 4, 8 within the 16-lane rows, then row_bcast:15 into rows 1
// and 3 and row_bcast:31 into rows 2 and 3), subtracted from the total.
__device__ __forceinline__ uint32_t wave_suffix_sum(uint32_t x) {
  uint32_t p = x;
  p += dpp_or_zero<0x111>(p);
  p += dpp_or_zero<0x112>(p);
  p += dpp_or_zero<0x114>(p);
  p += dpp_or_zero<0x118>(p);
  p += dpp_or_zero<0x142, 0xA>(p);
  p += dpp_or_zero<0x143, 0xC>(p);
  const uint32_t total = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(p), 63));
  return total - p + x;
}

// The lane whose bins hold the crossing walks them from the top.
template <int PER>
__device__ __forceinline__ void walk_bins(const uint32_t (&v)[PER], int tid, uint32_t excl, uint32_t need,
                                          uint32_t* s_res) {
  uint32_t c = excl;
  bool done = false;
#pragma unroll
  for (int i = PER - 1; i >= 0; --i) {
    if (!done && c + v[i] >= need) {
      s_res[0] = static_cast<uint32_t>(PER * tid + i);
      s_res[1] = c;
      s_res[2] = v[i];
      done = true;
    }
    c += v[i];
  }
}

// Block-wide (NT threads, NT * PER bins).  Every thread returns the result (and the count of
// bin t).  s_tot holds NT/64 words, s_res 3; both may be reused after the call.
template <int NT, int PER>
__device__ void block_threshold(const uint32_t* h, uint32_t need, uint32_t* s_tot, uint32_t* s_res, uint32_t& t_out,
                                uint32_t& above_out, uint32_t& count_out) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t v[PER];
  load_bins<PER>(h, tid, v);
  uint32_t sum = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) sum += v[i];
  const uint32_t suf = wave_suffix_sum(sum);
  if (lane == 0) s_tot[wv] = suf;
  __syncthreads();
  uint32_t higher = 0;
#pragma unroll
  for (int w2 = 0; w2 < NW; ++w2) higher += w2 > wv ? s_tot[w2] : 0u;
  const uint32_t incl = higher + suf, excl = incl - sum;
  if (excl < need && incl >= need) walk_bins<PER>(v, tid, excl, need, s_res);  // exactly one thread
  __syncthreads();
  t_out = s_res[0];
  above_out = s_res[1];
  count_out = s_res[2];
  __syncthreads();
}

// Redundant per-wave search of the top 64 * PER of NB bins: every wave that calls it reads the same
// bins and gets the same bin t (no LDS writes, no barrier).  False when those bins hold fewer than
// need (then t is untouched and the caller searches all bins).
template <int NB, int PER>
__device__ __forceinline__ bool wave_top_threshold(const uint32_t* h, uint32_t need, uint32_t& t_out) {
  constexpr int kLow = NB - 64 * PER;
  const int lane = threadIdx.x & 63;
  uint32_t v[PER];
  load_bins<PER>(h + kLow, lane, v);
  uint32_t sum = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) sum += v[i];
  const uint32_t incl = wave_suffix_sum(sum), excl = incl - sum;
  if (__builtin_amdgcn_readfirstlane(incl) < need) return false;  // lane 0's suffix is the total
  const uint64_t hit = __builtin_amdgcn_ballot_w64(excl < need && incl >= need);  // exactly one lane
  uint32_t t = 0u, c = excl;
  bool done = false;
#pragma unroll
  for (int i = PER - 1; i >= 0; --i) {
    if (!done && c + v[i] >= need) {
      t = static_cast<uint32_t>(PER * lane + i);
      done = true;
    }
    c += v[i];
  }
  t_out = kLow + static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(t), __builtin_ctzll(hit)));
  return true;
}

// Wave-only variant over 64 * PER bins (called by one whole wave); the result lands in s_res[0..2].
template <int PER>
__device__ void wave_threshold(const uint32_t* h, uint32_t need, uint32_t* s_res) {
  const int lane = threadIdx.x & 63;
  uint32_t v[PER];
  load_bins<PER>(h, lane, v);
  uint32_t sum = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) sum += v[i];
  const uint32_t incl = wave_suffix_sum(sum), excl = incl - sum;
  if (excl < need && incl >= need) walk_bins<PER>(v, lane, excl, need, s_res);
}

// ---- query side: rotation, digits, A fragments (once per workgroup, in LDS) --------------------
// Wave wv rotates heads wv + 4i (i < NRB); lane l holds elements l + 64e of the head.
// q~ = _wht(diag * q): stages h = 1..32 pair lanes (xor_lane), stage 64 pairs e = 0 and 1.  Then
// every lane assembles its A fragments (4 heads x 4 digits per row block) and combine constants.
//
// The query values, the diagonal and the head weights of a row, requested by query_loads for every
// row of the workgroup before any is used (one memory round; heads past IH read head 0's values).
template <int IC, int NRB>
struct QueryRaw {
  float q[NRB][IC / 64];
  float dg[IC / 64];
  float w[NRB];
};

template <int IC, int NRB>
__device__ __forceinline__ void query_loads(const MfmaIdxArgs& a, int b, QueryRaw<IC, NRB>& r) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int e = 0; e < IC / 64; ++e) r.dg[e] = a.diag[lane + 64 * e];
#pragma unroll
  for (int i = 0; i < NRB; ++i) {
    const int h = wv + 4 * i < a.IH ? wv + 4 * i : 0;
#pragma unroll
    for (int e = 0; e < IC / 64; ++e) r.q[i][e] = a.q[(static_cast<int64_t>(b) * a.IH + h) * IC + lane + 64 * e];
    r.w[i] = a.w[static_cast<int64_t>(b) * a.IH + h];
  }
}

// NWV: waves in the workgroup; waves 4 and up take no heads (they only build their fragments).
template <int BITS, int IC, int NRB, int NWV = 4>
__device__ __forceinline__ void query_fragments(const MfmaIdxArgs& a, const QueryRaw<IC, NRB>& raw,
                                                int8_t (*dig)[16][IC], float (*hf)[4], float (*hb)[2],
                                                i32x4_t (&A)[NRB][IC / 64], float (&f)[NRB][4], float (&lo)[NRB],
                                                float (&hi)[NRB]) {
  constexpr int KS = IC / 64;
  constexpr int EPL = IC / 64;
  const int IH = a.IH;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < NRB; ++i) {
    if (NWV > 4 && wv >= 4) break;  // wave-uniform
    const int h = wv + 4 * i;
    float v[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) v[e] = h < IH ? raw.q[i][e] * raw.dg[e] : 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float x = v[e];
      x = fmaf(x, (lane & 1) ? -1.0f : 1.0f, xor_lane<1>(x));    // lower lane: x + p, upper: p - x
      x = fmaf(x, (lane & 2) ? -1.0f : 1.0f, xor_lane<2>(x));
      x = fmaf(x, (lane & 4) ? -1.0f : 1.0f, xor_lane<4>(x));
      x = fmaf(x, (lane & 8) ? -1.0f : 1.0f, xor_lane<8>(x));
      x = fmaf(x, (lane & 16) ? -1.0f : 1.0f, xor_lane<16>(x));
      x = fmaf(x, (lane & 32) ? -1.0f : 1.0f, xor_lane<32>(x));
      v[e] = x;
    }
    if constexpr (EPL == 2) {
      const float x = v[0], y = v[1];
      v[0] = x + y;
      v[1] = x - y;
    }
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      v[e] = v[e] * a.wscale;
      mx = fmaxf(mx, fabsf(v[e]));
    }
    mx = wave_max(mx);
    // step S_h = 2^(e-6) from max|q~_h| = m * 2^e (m in [0.5, 1)); e >= -90 keeps every digit
    // step and its reciprocal normal
    int ex = 0;
    (void)frexpf(mx, &ex);
    ex = ex < -90 ? -90 : ex;
    const float step = mx > 0.0f ? ldexpf(1.0f, ex - 6) : 1.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float r = v[e];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float sd = ldexpf(step, -7 * d);
        const float di = rintf(r * (1.0f / sd));  // exact: 1/sd is a power of two
        r = fmaf(-di, sd, r);                      // exact residual
        dig[d][h][lane + 64 * e] = static_cast<int8_t>(di);
      }
    }
    // the head's weight (wave-uniform): read out before the lane-0 branch, so that its load is not
    // moved into that branch and given a wait of its own
    const float wr = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, raw.w[i])));
    if (lane == 0) {
      float wa = 0.0f, lw = -__builtin_inff(), hw = __builtin_inff();
      if (h < IH) {
        if (a.mode == AEKV_IDX_SOFTPLUS) {
          wa = softplus_f32(wr);
          lw = 0.0f;
        } else if (a.mode == AEKV_IDX_RAW) {
          wa = wr;
          if (wr >= 0.0f) lw = 0.0f; else hw = 0.0f;  // relu(dot)*w = clamp(dot*w) toward 0
        } else {
          wa = fmaxf(wr, 0.0f);                       // relu on the weight only
        }
      }
      const float unit = BITS == 4 ? 1.0f / 16.0f : 1.0f;
#pragma unroll
      for (int d = 0; d < 4; ++d) hf[h][d] = ldexpf(step, -7 * d) * unit * wa;
      hb[h][0] = lw;
      hb[h][1] = hw;
    }
  }
  __syncthreads();
  const int row = lane & 15;
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int h = 4 * rb + (row >> 2), d = row & 3;  // A rows = 4 heads x 4 digits
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
}

// ---- per-key scoring shared by the score kernel and the select's recomputation ---------------
// Raw code words of key j for lane group g (the B operand's k-step dims of the lane).
template <int BITS, int KS, int LW>
__device__ __forceinline__ void load_key_codes(const uint8_t* crow, uint32_t j, int g, uint32_t (&raw)[KS][LW]) {
  constexpr uint32_t RB = BITS == 8 ? 64 * KS : 32 * KS;  // code bytes per key
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if constexpr (BITS == 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(crow + (j * RB + 64 * ks + 16 * g));
      raw[ks][0] = v.x;
      raw[ks][1] = v.y;
      raw[ks][2] = v.z;
      raw[ks][3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(crow + (j * RB + 32 * ks + 8 * g));
      raw[ks][0] = v.x;
      raw[ks][1] = v.y;
    }
  }
}

// The B operand (int8 codes; 4-bit codes as 16 * code) of one 16-key block from its raw words.
template <int BITS, int KS, int LW>
__device__ __forceinline__ void build_bop(const uint32_t (&raw)[KS][LW], i32x4_t (&Bop)[KS]) {
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if constexpr (BITS == 8) {
      Bop[ks] = i32x4_t{static_cast<int>(raw[ks][0]), static_cast<int>(raw[ks][1]), static_cast<int>(raw[ks][2]),
                        static_cast<int>(raw[ks][3])};
    } else {
      const uint32_t x = raw[ks][0], y = raw[ks][1];
      Bop[ks] = i32x4_t{static_cast<int>((x << 4) & 0xF0F0F0F0u), static_cast<int>(x & 0xF0F0F0F0u),
                        static_cast<int>((y << 4) & 0xF0F0F0F0u), static_cast<int>(y & 0xF0F0F0F0u)};
    }
  }
}

// Score (before the key's scale) of lane l's key, key l % 16 of block l / 16 of the four blocks
// Bop[tq], for one row (A, f, lo, hi): the 4-head x 4-digit products, the digit pairs joined
// exactly in int32, the weights, the clamp, and the sum over heads (+ 0 turns -0 into +0, so that
// a zero score has one order key).
template <int NRB, int KS>
__device__ __forceinline__ float lane_score(const i32x4_t (&A)[NRB][KS], const i32x4_t (&Bop)[4][KS],
                                            const float (&f)[NRB][4], const float (&lo)[NRB], const float (&hi)[NRB]) {
  float tq_t[4];
#pragma unroll
  for (int tq = 0; tq < 4; ++tq) {
    i32x4_t acc[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) acc[rb] = i32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) acc[rb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[rb][ks], Bop[tq][ks], acc[rb], 0, 0, 0);
    float t = 0.0f;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      // f[d] = F 2^-7d: F (2^7 I_0 + I_1) 2^-7 + F (2^7 I_2 + I_3) 2^-21, the pairs exact in int32
      const int p01 = acc[rb][0] * 128 + acc[rb][1], p23 = acc[rb][2] * 128 + acc[rb][3];
      const float v = fmaf(static_cast<float>(p23), f[rb][3], static_cast<float>(p01) * f[rb][1]);
      const float m = __builtin_amdgcn_fmed3f(v, lo[rb], hi[rb]);
      t = rb == 0 ? m : t + m;
    }
    tq_t[tq] = t;
  }
  // sum over the four head groups; lane l keeps the key of block l / 16
  return row_sums_scatter(tq_t) + 0.0f;
}

// ---- score: keys -> order keys + the max of every 16-key slot ----------------------------------
// A wave scores groups of SPW slots of 64 keys; lane l keeps key base + 64s + l of slot s.  All
// loads of a group are issued before its matrix work.  With TT > 1 a workgroup scores TT rows
// of the same key row (prefill targets of one sequence) against every key group it loads: the
// codes and scales are read, and the integer B operand built, once for the TT rows.  Row
// (sequence bs, target t) is bs * T + t; workgroup row y takes targets TT (y % ceil(T / TT)) + tt.
// The register bound (at least 2 waves per SIMD, so at most 256 registers per lane) keeps the
// matrix results in VGPRs: with the default 512 the compiler uses the AGPR form and moves every
// result out with v_accvgpr_read.
template <int BITS, int IC, int NRB, int TT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void
idx_mfma_score_kernel(MfmaIdxArgs a) {
  touch_kernargs<sizeof(a)>();
  constexpr int KS = IC / 64;
  constexpr int RB = BITS == 8 ? IC : IC / 2;        // code bytes per key
  constexpr int SPW = score_spw(BITS, IC, TT);
  constexpr int LW = BITS == 8 ? 4 : 2;               // dwords per lane per k-step
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int64_t S = a.S;

  // this workgroup's rows: TT targets of key row kr (rows past the sequence's T are not scored)
  int64_t row[TT];
  bool rok[TT];
  int64_t kr;
  int64_t bx = blockIdx.x;  // key-range index
  if constexpr (TT == 1) {
    row[0] = blockIdx.y;
    rok[0] = true;
    // (32-bit: row < 65536, 1 <= T; a 64-bit division is a long emulated sequence ahead of the
    // first loads)
    kr = static_cast<uint32_t>(row[0]) / static_cast<uint32_t>(a.T);
  } else {
    // prefill: the linear workgroup ids are renumbered so that XCD x (linear id L runs on XCD
    // L % 8, each XCD with its own L2) runs the consecutive range [x n/8, (x+1) n/8) of (row group,
    // key range) pairs, i.e. whole sequences, whose keys then stay in that XCD's L2 for all of
    // their target groups
    int64_t by = blockIdx.y;
    const uint32_t nx = gridDim.x, n_wg = nx * gridDim.y;
    if (n_wg % 8 == 0) {
      const uint32_t L = blockIdx.y * nx + blockIdx.x;
      const uint32_t w = (L % 8) * (n_wg / 8) + L / 8;
      by = w / nx;
      bx = w % nx;
    }
    const int64_t ngt = (a.T + TT - 1) / TT;
    const uint32_t by32 = static_cast<uint32_t>(by), ngt32 = static_cast<uint32_t>(ngt);  // both < 65536
    kr = by32 / ngt32;
    const int64_t t0 = static_cast<int64_t>(by32 - static_cast<uint32_t>(kr) * ngt32) * TT;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      rok[tt] = t0 + tt < a.T;
      row[tt] = kr * a.T + (rok[tt] ? t0 + tt : t0);
    }
  }
  int64_t nv[TT], nv_max = 0;
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    // Prefill rows: unconditional scalar loads (uniform addresses, through the constant address
    // space), requested with the query's.  No select acts on a loaded value (the compiler turns such a
    // select into a branch around the load and waits for it where the branch joins, one target
    // after the other): the pointer is selected instead, a target past T reading kCountNone and a
    // launch without counts kCountAll.  Integer clamps (min<int64_t> lowers through doubles).
    // Decode rows (TT = 1) keep one vector load beside the query's (its address falls back on the
    // query's without counts; the constants' scalar load measured 0.1 us slower there).
    if constexpr (TT > 1) {
      const int32_t* vp = !rok[tt] ? &kCountNone : (a.valid ? a.valid + row[tt] : &kCountAll);
      const int32_t v = *(const __attribute__((address_space(4))) int32_t*)vp;
      nv[tt] = v <= 0 ? int64_t{0} : (v < S ? int64_t{v} : S);
    } else {
      nv[tt] = rok[tt] ? min<int64_t>(S, max(0, load_or(a.valid, row[tt], a.q, 0x7fffffff))) : 0;
    }
    nv_max = nv_max > nv[tt] ? nv_max : nv[tt];
  }

  __shared__ int8_t dig[4][16][IC];
  __shared__ float hf[16][4];  // per head: digit factors S * 2^-7d (/16 for 4-bit) * weight
  __shared__ float hb[16][2];  // per head: clamp bounds
  i32x4_t A[TT][NRB][KS];
  float f[TT][NRB][4], lo[TT][NRB], hi[TT][NRB];
  // key-row bases (wave-uniform) and 32-bit offsets within the rows (S <= kMaxKeys)
  const uint8_t* crow = a.codes + kr * S * RB;
  const uint8_t* srow = reinterpret_cast<const uint8_t*>(a.kscale + kr * S);
  constexpr int64_t kGroupKeys = SPW * 64;
  const int64_t wave_base = (bx * 4 + wv) * a.gpw * kGroupKeys;
  int nvi[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) nvi[tt] = static_cast<int>(nv[tt]);
  const int nv_maxi = static_cast<int>(nv_max);
  int nv_mini = nv_maxi;
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) nv_mini = min(nv_mini, nvi[tt]);
  // one group of SPW slots from key kb: its codes and scales (keys at or past lim read key 0;
  // CLAMP false: none is), then the scores; FULL: every key of the group is visible to every row
  // (no bounds checks)
  struct GroupRaw {
    uint32_t raw[SPW][4][KS][LW];
    float scl[SPW];
  };
  auto load_group = [&](const int kb, auto clamp_c, const int lim, GroupRaw& gr) {
    constexpr bool CLAMP = decltype(clamp_c)::value;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
#pragma unroll
      for (int tq = 0; tq < 4; ++tq) {
        const int j = kb + 64 * s + 16 * tq + (lane & 15);
        const uint32_t jr = !CLAMP || j < lim ? static_cast<uint32_t>(j) : 0u;
        load_key_codes<BITS, KS, LW>(crow, jr, g, gr.raw[s][tq]);
      }
      const int jo = kb + 64 * s + lane;
      gr.scl[s] = *reinterpret_cast<const float*>(srow + (!CLAMP || jo < lim ? static_cast<uint32_t>(jo) * 4u : 0u));
    }
  };
  // Decode rows (TT == 1) read their codes and scales through buffer resources whose ranges end at
  // the wave's last key (of the S stored, so that the first request does not wait for the row's
  // count): a load past it returns zeros without touching memory, so the next group is requested
  // unconditionally, while the current one is scored.
  const int64_t wkeys = max<int64_t>(0, min<int64_t>(wave_base + static_cast<int64_t>(a.gpw) * kGroupKeys, S) - wave_base);
  const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(crow + (wkeys > 0 ? wave_base * RB : 0)), 0, static_cast<int>(wkeys * RB), 0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(srow + (wkeys > 0 ? wave_base * 4 : 0)), 0, static_cast<int>(wkeys * 4), 0x00020000);
  auto fetch = [&](const int gi, GroupRaw& gr) {  // group gi of the wave (TT == 1)
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
#pragma unroll
      for (int tq = 0; tq < 4; ++tq) {
        const uint32_t j = static_cast<uint32_t>(gi * kGroupKeys + 64 * s + 16 * tq + (lane & 15));
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          if constexpr (BITS == 8) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(crs, j * RB + 64 * ks + 16 * g, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) gr.raw[s][tq][ks][e] = v[e];
          } else {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(crs, j * RB + 32 * ks + 8 * g, 0, 0);
            gr.raw[s][tq][ks][0] = v[0];
            gr.raw[s][tq][ks][1] = v[1];
          }
        }
      }
      gr.scl[s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                srs, static_cast<uint32_t>(gi * kGroupKeys + 64 * s + lane) * 4u, 0, 0));
    }
  };
  // The first memory round: the rows' counts (above), their queries and, for single-target rows, the
  // wave's first key group, which does not depend on the query (keys past S read key 0; those past
  // a row's count are dropped when scored).
  GroupRaw b0, b1;  // (TT == 1) the groups in flight
  {
    QueryRaw<IC, NRB> raw[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) query_loads<IC, NRB>(a, static_cast<int>(row[tt]), raw[tt]);
    if constexpr (TT == 1) fetch(0, b0);
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      if (tt > 0) __syncthreads();  // the previous row's fragments have been read out of LDS
      query_fragments<BITS, IC, NRB>(a, raw[tt], dig, hf, hb, A[tt], f[tt], lo[tt], hi[tt]);
    }
  }
  auto score_group = [&](const int kb, auto full_c, const GroupRaw& gr) {
    constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      i32x4_t Bop[4][KS];
#pragma unroll
      for (int tq = 0; tq < 4; ++tq) build_bop<BITS, KS, LW>(gr.raw[s][tq], Bop[tq]);
      const int jo = kb + 64 * s + lane;
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        if (!FULL && TT > 1 && kb + 64 * s >= nvi[tt]) continue;  // wave-uniform: this row has no key in the slot group
        const float mine = lane_score<NRB, KS>(A[tt], Bop, f[tt], lo[tt], hi[tt]);
        const bool ok = FULL || jo < nvi[tt];
        const uint32_t key = ok ? order_key(mine * gr.scl[s]) : 0u;
        uint8_t* krow = reinterpret_cast<uint8_t*>(a.keys + row[tt] * a.ks);
        uint8_t* mrow = reinterpret_cast<uint8_t*>(a.smax + row[tt] * a.ms);
        if (ok) *reinterpret_cast<uint32_t*>(krow + static_cast<uint32_t>(jo) * 4u) = key;
        // max of the 16-key slot of lanes 16u .. 16u+15: a prefix max along the row (row_shr by 1,
        // 2, 4, 8, lanes shifted in from outside the row read 0), stored by the row's last lane
        // when the slot's first key is visible (keys past the count are 0)
        uint32_t mx = key;
        mx = max(mx, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mx), 0x111, 0xF, 0xF, true)));
        mx = max(mx, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mx), 0x112, 0xF, 0xF, true)));
        mx = max(mx, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mx), 0x114, 0xF, 0xF, true)));
        mx = max(mx, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mx), 0x118, 0xF, 0xF, true)));
        if ((lane & 15) == 15 && (FULL || jo - 15 < nvi[tt]))
          *reinterpret_cast<uint32_t*>(mrow + static_cast<uint32_t>(jo >> 4) * 4u) = mx;
      }
    }
  };
  if constexpr (TT == 1) {
    // two groups in flight: group gi + 2 is requested as soon as group gi is scored (the
    // scheduling barriers keep each request batch in program order)
    __builtin_amdgcn_sched_barrier(0);
    fetch(1, b1);
    __builtin_amdgcn_sched_barrier(0);
    auto consume = [&](const int gi, const GroupRaw& gr) {
      const int64_t kb64 = wave_base + static_cast<int64_t>(gi) * kGroupKeys;
      if (gi >= a.gpw || kb64 >= nv_max) return;  // wave-uniform; past gpw are the next wave's keys
      if (kb64 + kGroupKeys <= nv_mini) score_group(static_cast<int>(kb64), std::true_type{}, gr);
      else score_group(static_cast<int>(kb64), std::false_type{}, gr);
    };
    // the first group's operands are built here, not hoisted above the query phase, where they
    // would hold registers
#pragma unroll
    for (int s2 = 0; s2 < SPW; ++s2)
#pragma unroll
      for (int tq = 0; tq < 4; ++tq)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int w = 0; w < LW; ++w) asm volatile("" : "+v"(b0.raw[s2][tq][ks][w]));
#pragma unroll 1
    for (int gi = 0; gi < a.gpw; gi += 2) {
      consume(gi, b0);
      __builtin_amdgcn_sched_barrier(0);
      fetch(gi + 2, b0);
      __builtin_amdgcn_sched_barrier(0);
      consume(gi + 1, b1);
      __builtin_amdgcn_sched_barrier(0);
      fetch(gi + 3, b1);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    auto group = [&](const int kb, auto full_c) {
      GroupRaw gr;
      // keys past a row's count read key 0 (nv_max >= 1 here) and are dropped
      load_group(kb, std::integral_constant<bool, !decltype(full_c)::value>{}, nv_maxi, gr);
      score_group(kb, full_c, gr);
    };
#pragma unroll 1
    for (int gi = 0; gi < a.gpw; ++gi) {
      const int64_t kb64 = wave_base + gi * kGroupKeys;
      if (kb64 >= nv_max) break;  // wave-uniform
      const bool full = kb64 + kGroupKeys <= nv_mini;
      if (full) group(static_cast<int>(kb64), std::true_type{});
      else group(static_cast<int>(kb64), std::false_type{});
    }
  }
}

// ---- final: exact top-k of a row, sorted ------------------------------------------------------
__device__ __forceinline__ uint64_t sort_word(uint32_t key, uint32_t idx) {
  // ascending order of (~key, idx) == key descending, index ascending
  return (static_cast<uint64_t>(~key) << 32) | idx;
}

// One workgroup per row.
//  1. Slot bound: every 16-key slot's max is one of its keys, so if kk slot maxima are >= tau
//     then the kk-th largest key is >= tau, and every top-kk key lies in a slot whose max is >=
//     tau.  tau is the floor of the bin holding the kk-th largest slot max in an LDS histogram of
//     the maxima whose 4096 bins are the values of key >> 16 just below the row's largest slot
//     max (1/128 of a binade each; the lowest bin also takes everything further down, and tau is
//     0 if it holds the kk-th).  Only the slots with max >= tau are read, and their keys >= tau
//     collected.
//  2. Three radix levels over the candidates (bits 31..20, 19..8, 7..0; LDS histograms) give
//     the kk-th largest key T; keys > T are taken with the lowest-index keys == T and the kk words
//     placed by rank.  If the candidates overflow LDS (many equal keys), the levels run over all
//     of the row's keys, read in index order.
// NT threads per row; CAP candidates collected in LDS; up to NT candidates sorted outright.
// 1024 / 4096 for few rows; 512 / 1536 (37 KB of LDS, at most 64 VGPRs: four rows per CU, where
// the 1024-thread instance fits one) for launches of many rows with k <= 512.
// sel_lds (nullable): the row's output indices also go there as int32 (-1 padding), for a caller
// that continues with them in the same workgroup.  during_wait: work of the caller's that needs no
// result of the select, run once, with the first slot maxima requested and not yet used (every
// thread of the workgroup calls it at the same point; rows with no visible block skip it).
// COLS: slot maxima each thread loads per pass (a pass covers COLS * NT slots); launches whose
// rows have at most 16 * COLS * NT keys take the smallest COLS that covers them, so that no thread
// issues loads that only fall past the row (each is an instruction through the CU's address unit
// in the workgroup's first memory round, and a register held until the list is built).
// Returns kk = min(k, visible count).
struct NoHook {
  __device__ void operator()() const {}
};

// nv: the row's visible count, visible(a, b), read by the caller (after requests of its own that
// do not depend on it).
template <int NT, int CAP, int COLS = kHistBins / NT, typename Hook = NoHook>
__device__ __forceinline__ uint32_t select_row(const MfmaIdxArgs& a, const int b, const int64_t nv,
                                               int64_t* __restrict__ out_idx, float* __restrict__ out_score,
                                               int32_t* __restrict__ sel_lds, Hook&& during_wait = Hook{}) {
  constexpr bool kHook = !std::is_same<std::decay_t<Hook>, NoHook>::value;
  constexpr int NW = NT / 64;
  __shared__ uint64_t cbuf[CAP];  // candidates: keys ck[] then indices ci[], or sort words
  __shared__ __align__(16) uint32_t h[kHistBins];
  __shared__ uint64_t sel[kMaxMfmaK];
  __shared__ uint32_t s_tot[NW], s_res[3], s_cnt[2], s_wave_eq[NW];
  uint32_t* ck = reinterpret_cast<uint32_t*>(cbuf);
  uint32_t* ci = ck + CAP;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int k = a.k;
  const uint32_t kk = static_cast<uint32_t>(min<int64_t>(k, nv));
  int64_t* orow = out_idx + static_cast<int64_t>(b) * k;
  float* srow = out_score ? out_score + static_cast<int64_t>(b) * k : nullptr;
  // the -1 padding past kk, written last (a store loop ahead of the loads below would make every
  // later wait for them wait for all of the workgroup's requests)
  auto pad = [&]() {
    for (int i = static_cast<int>(kk) + tid; i < k; i += NT) {
      orow[i] = -1;
      if (srow) srow[i] = -__builtin_inff();
      if (sel_lds) sel_lds[i] = -1;
    }
  };
  if (kk == 0) {
    pad();
    return 0u;
  }
  const uint32_t* krow = a.keys + static_cast<int64_t>(b) * a.ks;
  const uint32_t* mrow = a.smax + static_cast<int64_t>(b) * a.ms;
  const int64_t n_slots = (nv + 15) >> 4;
  // The row's slot maxima and order keys are read through buffer resources whose ranges end at its
  // last visible slot (S <= 2^24 keys: 32-bit offsets): a load past them returns 0 and touches no
  // memory, so the loads are branch-free and the wait counts exact.  (The count is read through the
  // vector unit; made scalar for the resources.)
  const int n_slots_i = __builtin_amdgcn_readfirstlane(static_cast<int>(n_slots));
  const __amdgpu_buffer_rsrc_t mrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(mrow), 0, n_slots_i * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(krow), 0, n_slots_i * 64, 0x00020000);

  // ---- 1. slot bound and candidates ----
  // thread tid owns slots c0 + tid + r * NT (r < kSlotPer) of each pass of kSlotPass slots; with
  // n_slots <= kSlotPass the maxima loaded for the histogram are reused for the scan
  static_assert(COLS >= 1 && COLS <= kHistBins / NT, "slot columns: 1 .. kHistBins / NT");
  constexpr int kSlotPer = COLS;  // one pass over the slot maxima for S <= 16 * COLS * NT
  constexpr int64_t kSlotPass = static_cast<int64_t>(kSlotPer) * NT;
  for (int i = tid; i < kHistBins; i += NT) h[i] = 0u;
  if (tid == 0) {
    s_cnt[0] = 0u;
    s_cnt[1] = 0u;
  }
  uint32_t mx[kSlotPer];
  auto load_max = [&](int64_t c0) {  // slots past the row read as 0
#pragma unroll
    for (int r = 0; r < kSlotPer; ++r)
      mx[r] = __builtin_amdgcn_raw_buffer_load_b32(mrs, static_cast<uint32_t>(c0 + tid + r * NT) * 4u, 0, 0);
  };
  // the row's largest slot max anchors the histogram
  uint32_t mloc = 0u;
  for (int64_t c0 = 0; c0 < n_slots; c0 += kSlotPass) {
    load_max(c0);
    if (kHook && c0 == 0) {
      __builtin_amdgcn_sched_barrier(0);  // the maxima are requested before the caller's work
      during_wait();
    }
#pragma unroll
    for (int r = 0; r < kSlotPer; ++r) mloc = mloc > mx[r] ? mloc : mx[r];  // mx is 0 past the end
  }
  mloc = wave_max_u32(mloc);
  if (lane == 0) s_tot[wv] = mloc;
  __syncthreads();  // also orders the zeroing of h before the histogram
  uint32_t top = 0u;
#pragma unroll
  for (int w2 = 0; w2 < NW; ++w2) top = top > s_tot[w2] ? top : s_tot[w2];
  top >>= 16;
  // slot columns r of a pass that hold a slot for some thread (workgroup-uniform): the work of
  // the others is skipped (a row of 1024 slots uses 2 of the 8 columns of 512 threads)
  auto columns = [&](int64_t c0) {
    return __builtin_amdgcn_readfirstlane(static_cast<int>(min<int64_t>(kSlotPer, (n_slots - c0 + NT - 1) / NT)));
  };
  // bin 4095 - d holds the maxima with key >> 16 == top - d (d < 4095); bin 0 everything lower
  for (int64_t c0 = 0; c0 < n_slots; c0 += kSlotPass) {
    if (n_slots > kSlotPass) load_max(c0);  // otherwise mx still holds the only pass
    const int n_col = columns(c0);
#pragma unroll
    for (int r = 0; r < kSlotPer; ++r) {
      if (r >= n_col) break;
      const uint32_t d = top - (mx[r] >> 16);
      if (tid + r * NT < n_slots_i - static_cast<int>(c0))
        atomicAdd(&h[kHistBins - 1 - (d < kHistBins - 1 ? d : kHistBins - 1)], 1u);
    }
  }
  __syncthreads();
  uint32_t tau = 0u;
  // Usually the kk-th largest slot max lies within 4 binades of the row's maximum: every wave finds
  // its bin among the top kTopBins bins by itself, and no barrier follows.  The list below is then
  // written to h while other waves may still read those bins, so it stays below them; a longer list
  // sends the row to the radix levels over all of its keys.
  constexpr int kTopBins = 512;
  constexpr int kListCap = kHistBins - kTopBins;
  bool list_cut = false;
  if (static_cast<int64_t>(kk) <= n_slots) {
    uint32_t t;
    if (!wave_top_threshold<kHistBins, kTopBins / 64>(h, kk, t)) {  // the same outcome in every wave
      uint32_t ab, ct;
      block_threshold<NT, kHistBins / NT>(h, kk, s_tot, s_res, t, ab, ct);
      (void)ab;
      (void)ct;
    }
    tau = t > 0u ? (top - (kHistBins - 1 - t)) << 16 : 0u;
  }
  // qualifying slots (max >= tau) are compacted into a list (in h, free until the radix levels),
  // then one thread per listed slot reads its 16 keys and appends those >= tau
  for (int64_t c0 = 0; c0 < n_slots; c0 += kSlotPass) {
    if (n_slots > kSlotPass) load_max(c0);  // otherwise mx still holds the only pass
    if (c0 > 0) {
      // a later pass: the previous pass's list (h) and count are free once every thread is here.
      // The first pass needs no barrier: s_cnt[1] was zeroed with s_cnt[0], and h's list part
      // [0, kListCap) is last read before the final barrier of block_threshold (or, when that is
      // skipped, last written before the histogram's barrier).
      __syncthreads();
      if (tid == 0) s_cnt[1] = 0u;
      __syncthreads();
    }
    {  // one reservation per wave for all of its slot columns
      const int n_col = columns(c0);
      bool q[kSlotPer];
      uint64_t m[kSlotPer];
      uint32_t tot = 0u;
#pragma unroll
      for (int r = 0; r < kSlotPer; ++r) {
        q[r] = false;
        m[r] = 0u;
        if (r >= n_col) continue;
        q[r] = tid + r * NT < n_slots_i - static_cast<int>(c0) && mx[r] >= tau;
        m[r] = __builtin_amdgcn_ballot_w64(q[r]);
        tot += static_cast<uint32_t>(__builtin_popcountll(m[r]));
      }
      uint32_t base = 0u;
      if (lane == 0 && tot != 0u) base = atomicAdd(&s_cnt[1], tot);
      base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
      for (int r = 0; r < kSlotPer; ++r) {
        if (r >= n_col) break;
        const uint32_t pos = base + static_cast<uint32_t>(mbcnt64(m[r]));
        if (q[r] && pos < static_cast<uint32_t>(kListCap)) h[pos] = static_cast<uint32_t>(tid + r * NT);
        base += static_cast<uint32_t>(__builtin_popcountll(m[r]));
      }
    }
    __syncthreads();
    list_cut = list_cut || s_cnt[1] > static_cast<uint32_t>(kListCap);
    const int n_list = min(static_cast<int>(s_cnt[1]), kListCap);
    for (int li = tid; li < n_list; li += NT) {
      const int64_t sl = c0 + h[li];
      uint32_t kw[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(krs, static_cast<uint32_t>(sl) * 64u + 16u * q, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) kw[4 * q + e] = v[e];
      }
      const int n_in = static_cast<int>(min<int64_t>(16, nv - 16 * sl));  // the slot's visible keys
      uint32_t qm = 0u;  // the slot's keys >= tau (about one per listed slot)
#pragma unroll
      for (int e = 0; e < 16; ++e) qm |= (e < n_in && kw[e] >= tau) ? (1u << e) : 0u;
      uint32_t p = wave_reserve<5>(&s_cnt[0], static_cast<uint32_t>(__builtin_popcount(qm)));  // <= 16
      // only the qualifying keys are visited (a loop over the set bits, not over all 16)
      while (qm != 0u) {
        const int e = __builtin_ctz(qm);
        qm &= qm - 1u;
        uint32_t ke = kw[0];
#pragma unroll
        for (int e2 = 1; e2 < 16; ++e2) ke = e == e2 ? kw[e2] : ke;  // (a select: no runtime index)
        if (p < static_cast<uint32_t>(CAP)) {
          ck[p] = ke;
          ci[p] = static_cast<uint32_t>(16 * sl + e);
        }
        ++p;
      }
    }
  }
  __syncthreads();
  const uint32_t n_cand = s_cnt[0];
  const bool fast = n_cand <= static_cast<uint32_t>(CAP) && !list_cut;
  const int n = fast ? static_cast<int>(n_cand) : 0;

  // ---- 2a. up to NT candidates (the usual case): sort them all, emit the first kk ----
  // Wave w sorts candidates 64w .. 64w+63 in registers (bitonic network over lane exchanges);
  // the runs go to LDS and every candidate's final position is its index in its run plus, for
  // each other run, the number of smaller words there (binary search).  Words are distinct.
  if (fast && n <= NT) {
    uint64_t w = tid < n ? sort_word(ck[tid], ci[tid]) : ~0ull;
    if (64 * wv < n) {  // wave-uniform: waves past the candidates only pad
#pragma unroll
      for (int kq = 2; kq <= 64; kq <<= 1) {
#pragma unroll
        for (int j = kq >> 1; j > 0; j >>= 1) {
          const uint64_t o = xor_lane_u64(w, j);
          const bool keep_min = ((lane & j) == 0) == ((lane & kq) == 0);
          // the smaller word on keep_min lanes, the larger on the others (words are distinct but
          // for the ~0 padding, where either is the same)
          w = (o < w) == keep_min ? o : w;
        }
      }
    }
    __syncthreads();  // ck/ci are read
    cbuf[tid] = w;    // run wv at cbuf[64 wv .. 64 wv + 63], ascending; runs past n_runs all ~0
    __syncthreads();
    const int n_runs = (n + 63) >> 6;
    if (tid < n) {
      // position = number of smaller words over all runs (the own run gives the lane); the binary
      // searches of up to 8 runs are interleaved so that their LDS reads overlap, and only the
      // runs that hold candidates are searched (the run count is workgroup-uniform)
      auto ranks = [&](auto nq_c) {
        constexpr int NQ = decltype(nq_c)::value;
        uint32_t pos = 0u;
        for (int r0 = 0; r0 < n_runs; r0 += NQ) {
          int lo[NQ];
#pragma unroll
          for (int q = 0; q < NQ; ++q) lo[q] = 0;
#pragma unroll
          for (int step = 32; step > 0; step >>= 1) {
#pragma unroll
            for (int q = 0; q < NQ; ++q)
              if (cbuf[64 * (r0 + q) + lo[q] + step - 1] < w) lo[q] += step;
          }
#pragma unroll
          for (int q = 0; q < NQ; ++q) {  // the steps reach 63; the last compare 64
            if (cbuf[64 * (r0 + q) + lo[q]] < w) ++lo[q];
            pos += static_cast<uint32_t>(lo[q]);
          }
        }
        return pos;
      };
      uint32_t pos;
      switch (__builtin_amdgcn_readfirstlane(n_runs)) {
        case 1: pos = ranks(std::integral_constant<int, 1>{}); break;
        case 2: pos = ranks(std::integral_constant<int, 2>{}); break;
        case 3: pos = ranks(std::integral_constant<int, 3>{}); break;
        case 4: pos = ranks(std::integral_constant<int, 4>{}); break;
        case 5: pos = ranks(std::integral_constant<int, 5>{}); break;
        case 6: pos = ranks(std::integral_constant<int, 6>{}); break;
        case 7: pos = ranks(std::integral_constant<int, 7>{}); break;
        default: pos = ranks(std::integral_constant<int, 8>{}); break;  // 8, or two passes and more
      }
      if (pos < kk) {
        orow[pos] = static_cast<int64_t>(static_cast<uint32_t>(w & 0xffffffffu));
        if (srow) srow[pos] = order_key_inv(~static_cast<uint32_t>(w >> 32));
        if (sel_lds) sel_lds[pos] = static_cast<int32_t>(w & 0xffffffffu);
      }
    }
    pad();
    return kk;
  }

  // ---- 2. three radix levels down to the kk-th largest key T ----
  uint32_t need = kk;  // keys still to take at or below the current prefix
  uint32_t prefix = 0u;
  int shift = 32;
#pragma unroll 1
  for (int lvl = 0; lvl < 3; ++lvl) {
    const int wbits = lvl < 2 ? 12 : 8;
    const int nb = 1 << wbits;
    const int nshift = shift - wbits;
    const uint32_t mask = static_cast<uint32_t>(nb - 1);
    __syncthreads();  // the previous level's readers of h are done
    for (int i = tid; i < nb; i += NT) h[i] = 0u;
    __syncthreads();
    // (key >> 32) is undefined: level 0 has no prefix to match
    if (fast) {
      for (int i = tid; i < n; i += NT) {
        const uint32_t key = ck[i];
        if (lvl == 0 || (key >> shift) == prefix) atomicAdd(&h[(key >> nshift) & mask], 1u);
      }
    } else {
      for (int64_t j = tid; j < nv; j += NT) {
        const uint32_t key = krow[j];
        if (lvl == 0 || (key >> shift) == prefix) atomicAdd(&h[(key >> nshift) & mask], 1u);
      }
    }
    __syncthreads();
    uint32_t t, ab, ct;
    if (lvl < 2) {
      block_threshold<NT, kHistBins / NT>(h, need, s_tot, s_res, t, ab, ct);
    } else {
      if (wv == 0) wave_threshold<4>(h, need, s_res);  // 256 bins
      __syncthreads();
      t = s_res[0];
      ab = s_res[1];
    }
    (void)ct;
    need -= ab;
    prefix = (prefix << wbits) | t;
    shift = nshift;
  }
  const uint32_t T = prefix;          // the kk-th largest key
  const uint32_t n_eq = h[T & 0xFFu]; // keys == T
  const uint32_t n_gt = kk - need;    // keys > T; `need` keys == T are taken, lowest index first
  __syncthreads();
  if (tid == 0) {
    s_cnt[0] = 0u;
    s_cnt[1] = 0u;
  }
  __syncthreads();
  if (fast) {
    const bool all_eq = n_eq == need;
    for (int i = tid; i < n; i += NT) {
      const uint32_t key = ck[i], idx = ci[i];
      const uint32_t pg = wave_reserve<1>(&s_cnt[0], key > T ? 1u : 0u);
      const uint32_t pe = wave_reserve<1>(&s_cnt[1], key == T && all_eq ? 1u : 0u);
      if (key > T) {
        if (pg < n_gt) sel[pg] = sort_word(key, idx);
      } else if (key == T) {
        if (all_eq) {
          if (pe < need) sel[n_gt + pe] = sort_word(key, idx);
        } else {  // ties at T: rank among the equal keys by index
          uint32_t r = 0;
          for (int j = 0; j < n; ++j) r += (ck[j] == T && ci[j] < idx) ? 1u : 0u;
          if (r < need) sel[n_gt + r] = sort_word(key, idx);
        }
      }
    }
  } else {
    uint32_t eq_run = 0;
    for (int64_t base = 0; base < nv; base += NT) {
      const int64_t j = base + tid;
      const uint32_t key = j < nv ? krow[j] : 0u;
      const bool gt = j < nv && key > T;
      const bool eq = j < nv && key == T;
      const uint32_t pg = wave_reserve<1>(&s_cnt[0], gt ? 1u : 0u);
      if (gt && pg < n_gt) sel[pg] = sort_word(key, static_cast<uint32_t>(j));
      const uint64_t m = __builtin_amdgcn_ballot_w64(eq);
      if (lane == 0) s_wave_eq[wv] = static_cast<uint32_t>(__builtin_popcountll(m));
      __syncthreads();
      uint32_t before = 0, total = 0;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) {
        const uint32_t c = s_wave_eq[w2];
        before += w2 < wv ? c : 0u;
        total += c;
      }
      if (eq) {
        const uint32_t r = eq_run + before + static_cast<uint32_t>(mbcnt64(m));
        if (r < need) sel[n_gt + r] = sort_word(key, static_cast<uint32_t>(j));
      }
      eq_run += total;
      __syncthreads();
    }
  }
  __syncthreads();
  // the kk words are distinct: each one's output position is its rank.  Four adjacent lanes
  // share an element, each counting over a quarter of the words.
  const int q4 = (static_cast<int>(kk) + 3) / 4;
  for (int base = 0; base < static_cast<int>(kk); base += NT / 4) {
    const int i = base + (tid >> 2), part = tid & 3;
    const uint64_t w = i < static_cast<int>(kk) ? sel[i] : 0ull;
    const int j0 = part * q4, j1 = min(static_cast<int>(kk), j0 + q4);
    uint32_t r = 0;
#pragma unroll 8
    for (int j = j0; j < j1; ++j) r += sel[j] < w ? 1u : 0u;
    r += __builtin_bit_cast(uint32_t, xor_lane<1>(__builtin_bit_cast(float, r)));
    r += __builtin_bit_cast(uint32_t, xor_lane<2>(__builtin_bit_cast(float, r)));
    if (part == 0 && i < static_cast<int>(kk)) {
      orow[r] = static_cast<int64_t>(static_cast<uint32_t>(w & 0xffffffffu));
      if (srow) srow[r] = order_key_inv(~static_cast<uint32_t>(w >> 32));
      if (sel_lds) sel_lds[r] = static_cast<int32_t>(w & 0xffffffffu);
    }
  }
  pad();
  return kk;
}

// The 512-thread instance serves launches of many rows: bounded to 64 VGPRs (eight waves per SIMD),
// so that four rows share a CU (it needs 57).
template <int NT, int CAP, int COLS>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT == 512 ? 8 : 1))) void idx_mfma_final_kernel(
    MfmaIdxArgs a, int64_t* __restrict__ out_idx, float* __restrict__ out_score) {
  touch_kernargs<sizeof(a) + 2 * sizeof(void*)>();
  select_row<NT, CAP, COLS>(a, blockIdx.x, visible(a, blockIdx.x), out_idx, out_score, nullptr);
}

// Whether every 16-key slot of rows of at most S keys lies within `cols` slot columns of NT
// threads (the select instance with COLS = cols then makes one pass over them).
__host__ __device__ constexpr bool slot_cols_fit(int64_t S, int NT, int cols) {
  return (S + 15) / 16 <= static_cast<int64_t>(cols) * NT;
}

// Launch set-up shared by the indexer and the fused CSA decode step: fills the kernel arguments
// for B rows (T per key row), enqueues the score kernel and returns its status.
int launch_mfma_score(MfmaIdxArgs& a, const float* q, const float* w, const void* codes, const float* kscale,
                      const float* diag, const int32_t* valid, int64_t B, int64_t T, int64_t S, int IH, int IC,
                      int bits, int k, int mode, void* ws, hipStream_t st, const char* who);

}  // namespace idx
}  // namespace aekv
