// Decode-step sink attention over TurboQuant-coded shared K=V blocks + a bf16 window, head_dim 128,
// with the QK^T and PV contractions on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16).
//
// Reference: aether_2b/serving.py:507-525 (HCA: every visible block) and :597-625 (CSA: the
// indexer's selected blocks), both followed by the sink attention of aether_pipeline/serving.py:
// 99-130 over [dequant(blocks), window] with K = V (serving.py:52-53).
//
// One workgroup (8 waves) owns a row (or a contiguous split of a long row's sources).  Per tile of 256
// sources it decodes the gathered code rows exactly (same code path as PolarQuant.decode, rounded
// to bf16 like the engine's dequantised cache) or copies window rows into an LDS tile, row-major.
// Wave w owns tile keys 32w..32w+31 and works transposed, so that each lane owns one head
// (lane & 15):
//   S^T = K Q^T        A = tile rows (16 keys x 32 dims), B = the row's queries;
//   online softmax of the lane's head over its 8 keys and across the 4 lane groups;
//   V^T blocks         the same A fragments times a 0/1 column selector (exact), which lands the
//                      values in the A layout of the next product with no LDS transpose;
//   O^T += V^T P^T     B = P^T straight from the softmax registers (bf16, the usual operand).
// The keys of a lane group appear in the same order in V^T and P^T, which is all the product
// needs.  The four waves' (max, sum, acc) are merged at the end; the sink joins the normaliser
// once, there or in the split combine.
#include <mutex>

#include "tq_device.h"

namespace aekv {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kD = 128;
constexpr int kTile = 32 * kWaves;     // sources per tile, 32 per wave
constexpr int kKP = kD + 8;            // row pitch of the staged tile (bf16)
constexpr int kMaxTilesPerSplit = 4;
constexpr float kNegInf = -__builtin_inff();

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

struct QAttnMfmaArgs {
  const uint16_t* q;      // [B, H, 128] bf16
  const uint8_t* codes;   // [B, S, 128 or 64]
  const float* scale;     // [B, S]
  const int64_t* sel;     // [B, K] or null (every block)
  const uint16_t* win;    // [B, W, 128] bf16
  const float* sink;      // [H]
  const float* diag;      // [128]
  int64_t S, K, W, n_comp, n_src;
  int H, n_split, tiles_per_split;
  float sm_scale, wscale;
  float* part;            // [B, n_split, H, 2 + 128] (split runs only)
  uint16_t* out;          // [B, H, 128] bf16
};

// LDS layout (bytes): staged tile | source flags | wave stats | the split's selected block ids
constexpr size_t kOffK = 0;
constexpr size_t kOffOk = kOffK + sizeof(uint16_t) * kTile * kKP;
constexpr size_t kOffSt = kOffOk + sizeof(float) * kTile;
constexpr size_t kOffIdx = kOffSt + sizeof(float) * kWaves * 16 * 2;
constexpr size_t kLds = kOffIdx + sizeof(int32_t) * kMaxTilesPerSplit * kTile;
static_assert(sizeof(float) * kWaves * 16 * kD <= kOffOk, "the wave merge reuses the staged tile");

__device__ __forceinline__ uint16_t bf16_bits(float v) { return static_cast<uint16_t>(pack_bf16x2(v, 0.0f) & 0xffffu); }

template <int BITS>
__global__ __launch_bounds__(kThreads) void quant_attn_mfma_kernel(QAttnMfmaArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];
  uint16_t* Kt = reinterpret_cast<uint16_t*>(lds + kOffK);
  float* okf = reinterpret_cast<float*>(lds + kOffOk);
  float* stat = reinterpret_cast<float*>(lds + kOffSt);  // [wave][head][m, l]
  constexpr int RB = BITS == 8 ? kD : kD / 2;

  const int64_t b = blockIdx.y;
  const int split = blockIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  const int H = a.H;

  // queries as the A operand: lane (head c16, group g) holds dims 32ks + 8g .. +7
  bf16x8_t qa[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (c16 < H) v = *reinterpret_cast<const uint4*>(a.q + (b * H + c16) * kD + 32 * ks + 8 * g);
    qa[ks] = __builtin_bit_cast(bf16x8_t, v);
  }
  // decode: the 16 lanes of group g hold dims 8*c16 .. +7 of one source
  float dg[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dg[e] = a.diag[8 * c16 + e];

  // softmax state and output of head c16 (replicated over the four lane groups)
  float m_run = kNegInf, l_run = 0.0f;
  f32x4_t O[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) O[nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // 0/1 selectors: esel[h] (lane column c16, element j of group g) = 1 iff 8g + j == c16 + 16h
  bf16x8_t esel[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k0 = 8 * g + 2 * e;
      w[e] = (k0 == c16 + 16 * h ? 0x3F80u : 0u) | (k0 + 1 == c16 + 16 * h ? 0x3F800000u : 0u);
    }
    esel[h] = __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
  }

  const int64_t n_tiles = (a.n_src + kTile - 1) / kTile;
  const int64_t t0 = static_cast<int64_t>(split) * a.tiles_per_split;
  const int64_t t1 = min<int64_t>(n_tiles, t0 + a.tiles_per_split);

  // block ids of this split's selected sources (-1: index outside [0, S), skipped)
  int32_t* sidx = reinterpret_cast<int32_t*>(lds + kOffIdx);
  const int64_t src0 = t0 * kTile;
  if (a.sel) {
    const int64_t nsel = min<int64_t>(t1 * kTile, a.n_comp) - src0;
    for (int64_t i = threadIdx.x; i < nsel; i += kThreads) {
      const int64_t blk = a.sel[b * a.K + src0 + i];
      sidx[i] = blk >= 0 && blk < a.S ? static_cast<int32_t>(blk) : -1;
    }
  }
  __syncthreads();

  // Staging of a tile: wave wv fills tile rows 32wv .. 32wv+31, four sources per pass (one per
  // 16-lane group).  The loads of a tile are issued together; kind: 0 empty, 1 code row, 2 window
  // row.
  constexpr int NB = LaneCodes<BITS, kD>::NB;  // code bytes per lane (4 or 8)
  uint32_t raw[8][4];
  float rsc[8];
  int kind[8];
  auto load_tile = [&](int64_t t) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int64_t si = t * kTile + 32 * wv + 4 * p + g;
      kind[p] = 0;
      raw[p][0] = raw[p][1] = raw[p][2] = raw[p][3] = 0u;
      rsc[p] = 0.0f;
      if (si < a.n_comp) {
        const int64_t blk = a.sel ? sidx[si - src0] : si;
        if (blk >= 0) {
          kind[p] = 1;
          const uint8_t* row = a.codes + (b * a.S + blk) * RB + c16 * NB;
          if constexpr (NB == 4) {
            raw[p][0] = *reinterpret_cast<const uint32_t*>(row);
          } else {
            const uint2 v = *reinterpret_cast<const uint2*>(row);
            raw[p][0] = v.x;
            raw[p][1] = v.y;
          }
          rsc[p] = a.scale[b * a.S + blk];
        }
      } else if (si < a.n_src) {
        kind[p] = 2;
        const uint4 v = *reinterpret_cast<const uint4*>(a.win + (b * a.W + (si - a.n_comp)) * kD + 8 * c16);
        raw[p][0] = v.x;
        raw[p][1] = v.y;
        raw[p][2] = v.z;
        raw[p][3] = v.w;
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int jj = 32 * wv + 4 * p + g;
      uint32_t w4[4] = {raw[p][0], raw[p][1], raw[p][2], raw[p][3]};
      if (kind[p] == 1) {  // uniform within the 16-lane group (one source)
        typename LaneCodes<BITS, kD>::type cb;
        __builtin_memcpy(cb.b, raw[p], NB);
        float v[8];
        decode_lane_bytes<BITS, kD>(cb, rsc[p], c16, dg, a.wscale, v);
#pragma unroll
        for (int e = 0; e < 4; ++e) w4[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
      }
      *reinterpret_cast<uint4*>(Kt + jj * kKP + 8 * c16) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
      if (c16 == 0) okf[jj] = kind[p] != 0 ? 1.0f : 0.0f;
    }
  };

#pragma unroll 1
  for (int64_t t = t0; t < t1; ++t) {
    load_tile(t);
    store_tile();
    __syncthreads();

    // ---- this wave's 32 keys: S^T = K Q^T, then O^T += V^T P^T ----
    // A fragments: kf[kb][ks] = K[key 32wv + 16kb + c16][dims 32ks + 8g .. +7]
    bf16x8_t kf[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        kf[kb][ks] = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const uint4*>(Kt + (32 * wv + 16 * kb + c16) * kKP + 32 * ks + 8 * g));
    // st[kb][i] = S[head c16][key 32wv + 16kb + 4g + i]
    f32x4_t st[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      st[kb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) st[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kb][ks], qa[ks], st[kb], 0, 0, 0);
    }
    // online softmax of head c16 over the wave's keys (8 per lane, 4 lane groups)
    float pr[2][4];
    {
      float lg[2][4];
      float tm = kNegInf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool ok = okf[32 * wv + 16 * kb + 4 * g + i] != 0.0f;
          lg[kb][i] = ok ? st[kb][i] * a.sm_scale : kNegInf;
          tm = fmaxf(tm, lg[kb][i]);
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
      // V columns 16nb .. 16nb+15 of the 32 keys: K rows times a 0/1 selector (exact)
      const f32x4_t v0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[0][nb >> 1], esel[nb & 1], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      const f32x4_t v1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[1][nb >> 1], esel[nb & 1], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      // A = V^T: lane (dim 16nb + c16), element 4kb + i <-> key 16kb + 4g + i (same order as pb)
      const bf16x8_t va = __builtin_bit_cast(
          bf16x8_t, make_uint4(pack_bf16x2(v0[0], v0[1]), pack_bf16x2(v0[2], v0[3]), pack_bf16x2(v1[0], v1[1]),
                               pack_bf16x2(v1[2], v1[3])));
      // O^T[nb][i] = O[head c16][dim 16nb + 4g + i]
      O[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, O[nb], 0, 0, 0);
    }
    __syncthreads();  // every wave is done with the tile before it is restaged
  }

  // ---- merge the waves (and the sink, unless this is one split of several) ----
  float* Ob = reinterpret_cast<float*>(lds);  // [wave][head][128]
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
  float* inv = okf;  // the source flags are no longer needed
  if (threadIdx.x < H) {
    const int h = threadIdx.x;
    float M = a.n_split == 1 ? a.sink[h] : kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, stat[(w * 16 + h) * 2]);
    float L = a.n_split == 1 ? __expf(a.sink[h] - M) : 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
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
  // every output: 4 consecutive dims per thread
  for (int p = threadIdx.x; p < H * (kD / 4); p += kThreads) {
    const int h = p / (kD / 4), d4 = 4 * (p % (kD / 4));
    f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = stat[(w * 16 + h) * 2];
      const f32x4_t o = *reinterpret_cast<const f32x4_t*>(Ob + (w * 16 + h) * kD + d4);
      acc = f32x4_t{fmaf(f, o[0], acc[0]), fmaf(f, o[1], acc[1]), fmaf(f, o[2], acc[2]), fmaf(f, o[3], acc[3])};
    }
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
// out = sum_s e^{m_s-M} acc_s / L.
__global__ __launch_bounds__(kThreads) void quant_attn_mfma_combine_kernel(QAttnMfmaArgs a) {
  const int64_t b = blockIdx.x;
  const int H = a.H, ns = a.n_split;
  const float* part = a.part + b * ns * H * (kD + 2);
  for (int p = threadIdx.x; p < H * kD; p += kThreads) {
    const int h = p / kD, d = p % kD;
    const float sk = a.sink[h];
    float M = sk;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, part[(s * H + h) * (kD + 2)]);
    float L = __expf(sk - M), acc = 0.0f;
    for (int s = 0; s < ns; ++s) {
      const float* ps = part + (s * H + h) * (kD + 2);
      const float ms = ps[0];
      const float f = ms == kNegInf ? 0.0f : __expf(ms - M);
      L = fmaf(f, ps[1], L);
      acc = fmaf(f, ps[2 + d], acc);
    }
    a.out[(b * H + h) * kD + d] = bf16_bits(acc / L);
  }
}

}  // namespace

bool quant_attn_mfma_supported(int64_t H, int64_t D) { return D == kD && H >= 1 && H <= 16; }

// Splits: one workgroup per row up to kMaxTilesPerSplit tiles (no combine); longer rows take
// kMaxTilesPerSplit tiles per workgroup and the split combine.
static int64_t split_count(int64_t n_tiles, int64_t& tiles_per_split) {
  tiles_per_split = n_tiles < kMaxTilesPerSplit ? n_tiles : kMaxTilesPerSplit;
  return tiles_per_split > 0 ? ceil_div(n_tiles, tiles_per_split) : 1;
}

size_t quant_attn_mfma_workspace(int64_t B, int64_t H, int64_t n_src) {
  int64_t tps = 1;
  const int64_t n_split = split_count(ceil_div(n_src, kTile), tps);
  return n_split > 1 ? align_up(static_cast<size_t>(B * n_split * H * (kD + 2)) * 4, 256) : 0;
}

int launch_quant_attn_mfma(const void* q, const void* codes, const float* scale, const int64_t* sel,
                           const void* window, const float* sink, const float* diag, int64_t B, int64_t H, int64_t S,
                           int64_t K, bool all_blocks, int64_t W, int bits, float softmax_scale, void* ws,
                           void* out, hipStream_t st, const char* who) {
  QAttnMfmaArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.codes = static_cast<const uint8_t*>(codes);
  a.scale = scale;
  a.sel = all_blocks ? nullptr : sel;
  a.win = static_cast<const uint16_t*>(window);
  a.sink = sink;
  a.diag = diag;
  a.S = S;
  a.K = K;
  a.W = W;
  a.n_comp = all_blocks ? S : K;
  a.n_src = a.n_comp + W;
  a.H = static_cast<int>(H);
  int64_t tps = 1;
  const int64_t n_split = split_count(ceil_div(a.n_src, kTile), tps);
  if (n_split > 65535) return fail(AEKV_ERR_UNSUPPORTED, "%s: too many sources", who);
  a.n_split = static_cast<int>(n_split);
  a.tiles_per_split = static_cast<int>(tps);
  a.sm_scale = softmax_scale;
  a.wscale = wht_scale(kD);
  a.part = static_cast<float*>(ws);
  a.out = static_cast<uint16_t*>(out);
  auto fn = bits == 8 ? quant_attn_mfma_kernel<8> : quant_attn_mfma_kernel<4>;
  static std::once_flag once8, once4;
  std::call_once(bits == 8 ? once8 : once4, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(kLds));
  });
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(n_split), static_cast<uint32_t>(B)), dim3(kThreads), kLds, st, a);
  if (int rc = check_launch(who)) return rc;
  if (n_split > 1) {
    hipLaunchKernelGGL(quant_attn_mfma_combine_kernel, dim3(static_cast<uint32_t>(B)), dim3(kThreads), 0, st, a);
    return check_launch(who);
  }
  return AEKV_OK;
}

}  // namespace aekv
