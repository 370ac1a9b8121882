// Decode-step sink attention over TurboQuant-coded shared K=V blocks + a bf16 window, head_dim 128,
// entirely on the matrix cores.
//
// Reference: aether_2b/serving.py:507-525 (HCA: every visible block) and :597-625 (CSA: the
// indexer's selected blocks), both followed by the sink attention of aether_pipeline/serving.py:
// 99-130 over [dequant(blocks), window] with K = V (serving.py:52-53).
//
// A workgroup (8 waves) owns a row, or a split of 1024 of a long row's sources.  Each wave takes
// groups of 32 sources (two blocks of 16 keys) and works in registers only:
//   dequantise  y = H128 codes on the int8 matrix cores (v_mfma_i32_16x16x64_i8), exact in int32:
//               H128 = [[H64, H64], [H64, -H64]], so two H64 products per 64-code half suffice;
//               4-bit codes enter as 16*code (the nibble shifted to the top of its byte).  Then
//               K = bf16(y * scale * c) — the engine attends the bf16 dequantised cache; this
//               differs from PolarQuant.decode's fp32 butterfly rounding by at most one bf16 ulp,
//               and only where y*scale*c lies within ~1e-7 relative of a bf16 rounding boundary.
//               The +-1 diagonal is folded into the queries and the output (bf16 rounding is
//               sign-symmetric), window rows get it on load.
//   S^T = K Q^T  (v_mfma_f32_16x16x32_bf16): A = the keys as decoded (lane = key), B = queries;
//               each lane then owns one head (lane & 15).
//   online softmax of the lane's head over its 8 keys and across the 4 lane groups;
//   V^T blocks   the same K fragments times a 0/1 column selector (exact), landing in the A layout
//               of O^T += V^T P^T, whose B = P^T comes straight from the softmax registers.
// Waves never share data inside the loop; their (max, sum, acc) are merged at the end, where the
// sink joins the normaliser once (or in the split combine).
#include <mutex>

#include "tq_device.h"

namespace aekv {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kD = 128;
constexpr int kGroup = 32;                    // sources per wave step
constexpr int kSplitSrc = 1024;               // most sources per workgroup (a row is split beyond)
#ifndef AEKV_ATTN_MIN_SPLIT
#define AEKV_ATTN_MIN_SPLIT 512
#endif
#ifndef AEKV_ATTN_TARGET_WG
#define AEKV_ATTN_TARGET_WG 512
#endif
constexpr float kNegInf = -__builtin_inff();

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) int i32x4_t;

struct QAttnMfmaArgs {
  const uint16_t* q;      // [B, H, 128] bf16
  const uint8_t* codes;   // [B, S, 128 or 64]
  const float* scale;     // [B, S]
  const int64_t* sel;     // [B, K] or null (every block)
  const uint16_t* win;    // [B / T, Wt, 128] bf16
  const float* sink;      // [H]
  const float* diag;      // [128]
  // Rows are targets: row r reads cache row r / T (codes, scale, window); q, sel, out are per row.
  // Per-row sources: vis[r] compressed blocks (null: n_comp), window entries
  // [wstart[r], wstart[r] + wlen[r]) of its cache row (null: wstart 0, wlen to the end of the
  // Wt entries); all clamped to the buffers.
  const int32_t* vis;
  const int32_t* wstart;
  const int32_t* wlen;
  int64_t T, Wt;
  int64_t S, K, n_comp, n_src;
  int H, n_split, split_src;
  float sm_scale, wscale;
  float* part;            // [B, n_split, H, 2 + 128] (split runs only)
  uint16_t* out;          // [B, H, 128] bf16
};

// LDS layout (bytes) for NW waves: wave outputs for the merge | wave stats | per-head factors |
// block ids
template <int NW>
struct QLay {
  static constexpr size_t ob = 0;
  static constexpr size_t st = ob + sizeof(float) * NW * 16 * kD;
  static constexpr size_t inv = st + sizeof(float) * NW * 16 * 2;
  static constexpr size_t idx = inv + sizeof(float) * 16;
  static constexpr size_t bytes = idx + sizeof(int32_t) * kSplitSrc;
};

__device__ __forceinline__ uint16_t bf16_bits(float v) { return static_cast<uint16_t>(pack_bf16x2(v, 0.0f) & 0xffffu); }

// Code index (within a 64-code half) of element p of lane group g's 16-byte operand, matching how
// the codes are loaded: 8-bit in byte order; 4-bit as (w << 4) & 0xF0F0F0F0 (even codes) and
// w & 0xF0F0F0F0 (odd codes) for each of the lane's two code dwords.
template <int BITS>
__device__ __forceinline__ int code_index(int g, int p) {
  if constexpr (BITS == 8) {
    return 16 * g + p;
  } else {
    const int q4 = p >> 2, r = p & 3;
    return 16 * g + 8 * (q4 >> 1) + 2 * r + (q4 & 1);
  }
}

// NW waves per workgroup: 8 for few rows (more waves share a row's sources), 4 for launches with
// many rows (prefill), where half the merge work and LDS lets twice the workgroups reside.
template <int BITS, int NW>
__global__ __launch_bounds__(64 * NW) void quant_attn_mfma_kernel(QAttnMfmaArgs a) {
  constexpr int kW = NW, kT = 64 * NW;
  using L = QLay<NW>;
  extern __shared__ __align__(16) unsigned char lds[];
  float* Ob = reinterpret_cast<float*>(lds + L::ob);    // [wave][head][128]
  float* stat = reinterpret_cast<float*>(lds + L::st);  // [wave][head][m, l]
  float* inv = reinterpret_cast<float*>(lds + L::inv);  // [head]
  int32_t* sidx = reinterpret_cast<int32_t*>(lds + L::idx);
  constexpr int RB = BITS == 8 ? kD : kD / 2;   // code bytes per row
  constexpr int HB = RB / 2;                    // code bytes per 64-code half

  const int64_t b = blockIdx.y;
  const int split = blockIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  const int H = a.H;

  // the row's sources: n_comp compressed blocks, then wl window entries from w0 of its cache row
  const int64_t cb = b / a.T;
  const int64_t n_comp = a.vis ? min<int64_t>(max(a.vis[b], 0), a.n_comp) : a.n_comp;
  const int64_t w0 = a.wstart ? min<int64_t>(max(a.wstart[b], 0), a.Wt) : 0;
  const int64_t wl = a.wlen ? min<int64_t>(max(a.wlen[b], 0), a.Wt - w0) : a.Wt - w0;
  // this workgroup's sources [src0, src1); the selected block ids go to LDS (-1: skipped)
  const int64_t src0 = static_cast<int64_t>(split) * a.split_src;
  const int64_t src1 = min<int64_t>(n_comp + wl, src0 + a.split_src);
  if (a.sel) {
    const int64_t nsel = min<int64_t>(src1, n_comp) - src0;
    for (int64_t i = threadIdx.x; i < nsel; i += kT) {
      const int64_t blk = a.sel[b * a.K + src0 + i];
      sidx[i] = blk >= 0 && blk < a.S ? static_cast<int32_t>(blk) : -1;
    }
  }

  // The lane's 32 dims, for every key it holds: element j of k-step ks (bf16x8) is dim
  // 16*(2ks + (j >> 2)) + 4g + (j & 3).  dsign: the diagonal's sign bits for those dims, per
  // packed bf16 pair (dword e of k-step ks).
  uint32_t dsign[4][4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d0 = 16 * (2 * ks + (e >> 1)) + 4 * g + 2 * (e & 1);
      dsign[ks][e] = (a.diag[d0] < 0.0f ? 0x8000u : 0u) | (a.diag[d0 + 1] < 0.0f ? 0x80000000u : 0u);
    }
  // queries (times the diagonal) as the B operand of S^T: lane (head c16), the lane's dims
  bf16x8_t qb[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint2 lo = make_uint2(0u, 0u), hi = make_uint2(0u, 0u);
    if (c16 < H) {
      const uint16_t* qr = a.q + (b * H + c16) * kD + 4 * g;
      lo = *reinterpret_cast<const uint2*>(qr + 16 * (2 * ks));
      hi = *reinterpret_cast<const uint2*>(qr + 16 * (2 * ks + 1));
    }
    qb[ks] = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x ^ dsign[ks][0], lo.y ^ dsign[ks][1], hi.x ^ dsign[ks][2],
                                                     hi.y ^ dsign[ks][3]));
  }
  // H64 rows 16a + c16 as int8 +-1 over the lane's code indices (the A operand of the dequantise)
  i32x4_t hA[4];
#pragma unroll
  for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
    for (int dw = 0; dw < 4; ++dw) {
      uint32_t word = 0;
#pragma unroll
      for (int by = 0; by < 4; ++by) {
        const int c = code_index<BITS>(g, 4 * dw + by);
        const bool neg = __builtin_popcount(static_cast<unsigned>((16 * a4 + c16) & c)) & 1;
        word |= (neg ? 0xFFu : 0x01u) << (8 * by);
      }
      hA[a4][dw] = static_cast<int>(word);
    }
  // 0/1 selectors: esel[h] (lane column c16, element j of group g) = 1 iff g == c16 >> 2 and
  // j == (c16 & 3) + 4h, i.e. column c16 picks dim 16*(2ks + h) + c16 of k-step ks
  bf16x8_t esel[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j0 = 2 * e;
      const bool mine = g == (c16 >> 2);
      w[e] = (mine && j0 == (c16 & 3) + 4 * h ? 0x3F80u : 0u) | (mine && j0 + 1 == (c16 & 3) + 4 * h ? 0x3F800000u : 0u);
    }
    esel[h] = __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
  }
  __syncthreads();  // sidx

  // softmax state and output of head c16 (replicated over the four lane groups)
  float m_run = kNegInf, l_run = 0.0f;
  f32x4_t O[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) O[nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const float kscale_unit = (BITS == 4 ? 1.0f / 16.0f : 1.0f) * a.wscale;

  const int n_groups = src1 > src0 ? static_cast<int>((src1 - src0 + kGroup - 1) / kGroup) : 0;
#pragma unroll 1
  for (int G = wv; G < n_groups; G += kW) {
    // both blocks' rows are requested before either is decoded (two gathers in flight)
    int kind[2];  // 0 empty, 1 code row, 2 window row
    uint32_t cw[2][2][BITS == 8 ? 4 : 2];
    float sraw[2];
    uint2 wv2[2][4][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      // lane (key c16 of block kb): its source, code bytes (two halves) or window dims
      const int64_t si = src0 + static_cast<int64_t>(G) * kGroup + 16 * kb + c16;
      kind[kb] = 0;
      int64_t blk = -1;
      if (si < n_comp) {
        blk = a.sel ? sidx[si - src0] : si;
        kind[kb] = blk >= 0 ? 1 : 0;
      } else if (si < src1) {
        kind[kb] = 2;
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int e = 0; e < (BITS == 8 ? 4 : 2); ++e) cw[kb][hh][e] = 0u;
      sraw[kb] = 0.0f;
      if (kind[kb] == 1) {
        const uint8_t* row = a.codes + (cb * a.S + blk) * RB;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          if constexpr (BITS == 8) {
            const uint4 v = *reinterpret_cast<const uint4*>(row + HB * hh + 16 * g);
            cw[kb][hh][0] = v.x;
            cw[kb][hh][1] = v.y;
            cw[kb][hh][2] = v.z;
            cw[kb][hh][3] = v.w;
          } else {
            const uint2 v = *reinterpret_cast<const uint2*>(row + HB * hh + 8 * g);
            cw[kb][hh][0] = v.x;
            cw[kb][hh][1] = v.y;
          }
        }
        sraw[kb] = a.scale[cb * a.S + blk];
      }
      if (kind[kb] == 2) {
        const uint16_t* wr = a.win + (cb * a.Wt + w0 + (si - n_comp)) * kD + 4 * g;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          wv2[kb][ks][0] = *reinterpret_cast<const uint2*>(wr + 16 * (2 * ks));
          wv2[kb][ks][1] = *reinterpret_cast<const uint2*>(wr + 16 * (2 * ks + 1));
        }
      }
    }

    bf16x8_t kf[2][4];
    bool okk[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      okk[kb] = kind[kb] != 0;
      const float fk = sraw[kb] * kscale_unit;
      // y = H64 codes per half (all lanes take part; lanes without a code row supply zeros)
      i32x4_t P[2][4];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        i32x4_t Bop;
        if constexpr (BITS == 8) {
          Bop = i32x4_t{static_cast<int>(cw[kb][hh][0]), static_cast<int>(cw[kb][hh][1]),
                        static_cast<int>(cw[kb][hh][2]), static_cast<int>(cw[kb][hh][3])};
        } else {
          const uint32_t x = cw[kb][hh][0], y = cw[kb][hh][1];
          Bop = i32x4_t{static_cast<int>((x << 4) & 0xF0F0F0F0u), static_cast<int>(x & 0xF0F0F0F0u),
                        static_cast<int>((y << 4) & 0xF0F0F0F0u), static_cast<int>(y & 0xF0F0F0F0u)};
        }
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4)
          P[hh][a4] = __builtin_amdgcn_mfma_i32_16x16x64_i8(hA[a4], Bop, i32x4_t{0, 0, 0, 0}, 0, 0, 0);
      }
      // P[hh][a4][i] = (H64 codes_half_hh)[16*a4 + 4g + i]; dims 16*blk + 4g + i of the full
      // transform: blk < 4 -> P[0] + P[1], blk >= 4 -> P[0] - P[1]
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        uint32_t w4[4];
        if (kind[kb] == 2) {
          w4[0] = wv2[kb][ks][0].x ^ dsign[ks][0];
          w4[1] = wv2[kb][ks][0].y ^ dsign[ks][1];
          w4[2] = wv2[kb][ks][1].x ^ dsign[ks][2];
          w4[3] = wv2[kb][ks][1].y ^ dsign[ks][3];
        } else {
          float v[8];
#pragma unroll
          for (int hv = 0; hv < 2; ++hv) {
            const int blk8 = 2 * ks + hv;
            const int a4 = blk8 & 3;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int y = blk8 < 4 ? P[0][a4][i] + P[1][a4][i] : P[0][a4][i] - P[1][a4][i];
              v[4 * hv + i] = static_cast<float>(y) * fk;
            }
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) w4[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
        }
        kf[kb][ks] = __builtin_bit_cast(bf16x8_t, make_uint4(w4[0], w4[1], w4[2], w4[3]));
      }
    }

    // st[kb][i] = S[head c16][key 16kb + 4g + i of the group]
    f32x4_t st[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      st[kb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) st[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kb][ks], qb[ks], st[kb], 0, 0, 0);
    }
    float pr[2][4];
    {
      float lg[2][4];
      float tm = kNegInf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        // okk[kb] belongs to key c16, so bit 4g+i of its ballot is the validity of row 4g+i
        const uint64_t okm = __builtin_amdgcn_ballot_w64(okk[kb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool ok = (okm >> (4 * g + i)) & 1u;
          lg[kb][i] = ok ? st[kb][i] * a.sm_scale : kNegInf;
          tm = fmaxf(tm, lg[kb][i]);
        }
      }
      tm = fmaxf(tm, xor_lane<16>(tm));
      tm = fmaxf(tm, xor_lane<32>(tm));
      const float mnew = fmaxf(m_run, tm);
      const float corr = m_run == kNegInf ? 0.0f : __expf(m_run - mnew);
      float ps = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[kb][i] = lg[kb][i] == kNegInf ? 0.0f : __expf(lg[kb][i] - mnew);
          ps += pr[kb][i];
        }
      ps += xor_lane<16>(ps);
      ps += xor_lane<32>(ps);
      l_run = l_run * corr + ps;
      m_run = mnew;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) O[nb] *= corr;
    }
    // B = P^T: lane (head c16), element 4kb + i <-> key 16kb + 4g + i
    const bf16x8_t pb = __builtin_bit_cast(
        bf16x8_t, make_uint4(pack_bf16x2(pr[0][0], pr[0][1]), pack_bf16x2(pr[0][2], pr[0][3]),
                             pack_bf16x2(pr[1][0], pr[1][1]), pack_bf16x2(pr[1][2], pr[1][3])));
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      // V columns 16nb .. 16nb+15 of the 32 keys: K fragments times a 0/1 selector (exact)
      const f32x4_t v0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[0][nb >> 1], esel[nb & 1], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      const f32x4_t v1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[1][nb >> 1], esel[nb & 1], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      // A = V^T: lane (dim 16nb + c16), element 4kb + i <-> key 16kb + 4g + i (same order as pb)
      const bf16x8_t va = __builtin_bit_cast(
          bf16x8_t, make_uint4(pack_bf16x2(v0[0], v0[1]), pack_bf16x2(v0[2], v0[3]), pack_bf16x2(v1[0], v1[1]),
                               pack_bf16x2(v1[2], v1[3])));
      // O^T[nb][i] = O[head c16][dim 16nb + 4g + i] (times diag, removed at the end)
      O[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, O[nb], 0, 0, 0);
    }
  }

  // ---- merge the waves (and the sink, unless this is one split of several) ----
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
    *reinterpret_cast<f32x4_t*>(Ob + (wv * 16 + c16) * kD + 16 * nb + 4 * g) = O[nb];
  if (g == 0) {
    stat[(wv * 16 + c16) * 2] = m_run;
    stat[(wv * 16 + c16) * 2 + 1] = l_run;
  }
  __syncthreads();
  // per head (one thread each): M = max(sink, wave maxima), the waves' factors e^{m_w - M}, and
  // the normaliser L; the factors replace the maxima in stat, 1/L (or L for a split) is kept aside
  if (threadIdx.x < H) {
    const int h = threadIdx.x;
    float M = a.n_split == 1 ? a.sink[h] : kNegInf;
#pragma unroll
    for (int w = 0; w < kW; ++w) M = fmaxf(M, stat[(w * 16 + h) * 2]);
    float L = a.n_split == 1 ? __expf(a.sink[h] - M) : 0.0f;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const float mw = stat[(w * 16 + h) * 2];
      const float f = mw == kNegInf ? 0.0f : __expf(mw - M);
      L = fmaf(f, stat[(w * 16 + h) * 2 + 1], L);
      stat[(w * 16 + h) * 2] = f;
    }
    if (a.n_split == 1) {
      inv[h] = 1.0f / L;
    } else {
      float* dst = a.part + ((b * a.n_split + split) * H + h) * (kD + 2);
      dst[0] = M;
      dst[1] = L;
    }
  }
  __syncthreads();
  // every output: 4 consecutive dims per thread; the diagonal folded into the keys comes off here
  for (int p = threadIdx.x; p < H * (kD / 4); p += kT) {
    const int h = p / (kD / 4), d4 = 4 * (p % (kD / 4));
    f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const float f = stat[(w * 16 + h) * 2];
      const f32x4_t o = *reinterpret_cast<const f32x4_t*>(Ob + (w * 16 + h) * kD + d4);
      acc = f32x4_t{fmaf(f, o[0], acc[0]), fmaf(f, o[1], acc[1]), fmaf(f, o[2], acc[2]), fmaf(f, o[3], acc[3])};
    }
    const float4 dg = *reinterpret_cast<const float4*>(a.diag + d4);
    acc = f32x4_t{acc[0] * dg.x, acc[1] * dg.y, acc[2] * dg.z, acc[3] * dg.w};
    if (a.n_split == 1) {
      const float r = inv[h];
      const uint2 v = make_uint2(pack_bf16x2(acc[0] * r, acc[1] * r), pack_bf16x2(acc[2] * r, acc[3] * r));
      *reinterpret_cast<uint2*>(a.out + (b * H + h) * kD + d4) = v;
    } else {
      float* dst = a.part + ((b * a.n_split + split) * H + h) * (kD + 2) + 2 + d4;
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e] = acc[e];
    }
  }
}

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

}  // namespace

// Sources per workgroup: kSplitSrc, halved (down to AEKV_ATTN_MIN_SPLIT) while the grid has fewer
// than AEKV_ATTN_TARGET_WG workgroups, so that few long rows still spread over the chip.  A row
// with more sources than that takes one workgroup per piece plus the split combine.
int64_t split_sources(int64_t rows, int64_t n_src) {
  int64_t s = kSplitSrc;
  while (s > AEKV_ATTN_MIN_SPLIT && rows * ceil_div(std::max<int64_t>(n_src, 1), s) < AEKV_ATTN_TARGET_WG) s >>= 1;
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
