// Sink attention kernels for gfx950.
//
// 1. sparse_attn_kernel — drop-in for sparse_sink_attention (aether_kernels/sparse_attention.py:8-16,
//    semantics aether_kernels/csrc/sparse_sink_attention_cuda.cu:47-114, oracle
//    aether_pipeline/serving.py:99-130) and, with dense indices, for tiled_prefill_attention
//    (aether_kernels/sparse_attention.py:19-42) with the sink counted once as in
//    aether_2b/modeling.py:158-178, for fp32 inputs and head dims other than 128 (bf16/fp16 at
//    head_dim 128 run on the matrix cores, sink_attention_mfma.hip).  One wave per (b, t, h); keys
//    streamed in tiles of 64 with an online softmax; the sink joins the normaliser once at the end.
// 2. quant_attn_partial_kernel + quant_attn_combine_kernel — one decode token per row over
//    TurboQuant-compressed shared K=V blocks (selected by the CSA indexer, or all blocks for HCA)
//    plus a bf16 sliding window (aether_2b/serving.py:507-522, :597-625).  Split-KV: each workgroup
//    gathers one tile of sources, dequantises the code rows on load to the same bf16 values
//    PolarQuant.decode produces, attends them for all heads of the row and writes (max, sum, acc);
//    the combine merges the tiles with the sink counted once.
// 3. hca_compress_kernel — softmax over the M window positions and weighted sum
//    (aether_kernels/sparse_attention.py:70-83; aether_2b/serving.py:495-497).
#include <mutex>
#include <unordered_set>

#include "tq_device.h"

namespace aekv {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 64;           // keys per online-softmax step in sparse_attn_kernel
constexpr int kMaxD = 512;
constexpr int kTileFloats = 8192;   // source tile of quant_attn_partial_kernel (32 KB)
constexpr float kNegInf = -__builtin_inff();

template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  if constexpr (DT == AEKV_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == AEKV_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
  if constexpr (DT == AEKV_F32) static_cast<float*>(p)[i] = v;
  else if constexpr (DT == AEKV_BF16) static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(pack_bf16x2(v, 0.0f) & 0xffffu);
  else static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_f16_bits(v));
}

// ------------------------------------------------------------------------------------------
// 1. general sparse sink attention
// ------------------------------------------------------------------------------------------
template <int DT, int IDX>  // IDX: 0 dense (index = position), 4 int32, 8 int64
__global__ __launch_bounds__(kThreads) void sparse_attn_kernel(const void* __restrict__ q, const void* __restrict__ kv,
                                                               const void* __restrict__ idx,
                                                               const void* __restrict__ sink, int sink_scalar,
                                                               int64_t rows, int64_t T, int64_t H, int D, int64_t S,
                                                               int64_t K, float scale, void* __restrict__ out) {
  __shared__ float qsh[kThreads / 64][kMaxD];
  __shared__ float psh[kThreads / 64][kTile];
  __shared__ int64_t ish[kThreads / 64][kTile];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + w;  // (b, t, h) flattened
  if (row >= rows) return;  // wave-uniform
  const int64_t h = row % H;
  const int64_t bt = row / H;
  const int64_t b = bt / T;
  for (int d = lane; d < D; d += 64) qsh[w][d] = ld<DT>(q, row * D + d);
  const float sk = ld<DT>(sink, sink_scalar ? 0 : h);
  constexpr int kMaxDPL = kMaxD / 64;
  float acc[kMaxDPL];
#pragma unroll
  for (int i = 0; i < kMaxDPL; ++i) acc[i] = 0.0f;
  float m = kNegInf, l = 0.0f;
  __builtin_amdgcn_wave_barrier();

  for (int64_t j0 = 0; j0 < K; j0 += kTile) {
    const int64_t j = j0 + lane;
    int64_t src = -1;
    if (j < K) {
      if constexpr (IDX == 0) src = j;
      else if constexpr (IDX == 4) src = static_cast<const int32_t*>(idx)[bt * K + j];
      else src = static_cast<const int64_t*>(idx)[bt * K + j];
    }
    float logit = kNegInf;
    if (src >= 0 && src < S) {
      const int64_t kbase = ((b * S + src) * 2 + 0) * D;
      float dot = 0.0f;
      for (int d = 0; d < D; ++d) dot = fmaf(qsh[w][d], ld<DT>(kv, kbase + d), dot);
      logit = dot * scale;
    } else {
      src = -1;
    }
    const float tmax = wave_max(logit);
    const float mnew = fmaxf(m, tmax);
    const float p = (src >= 0) ? __expf(logit - mnew) : 0.0f;
    const float corr = (m == kNegInf) ? 0.0f : __expf(m - mnew);
    l = l * corr + wave_sum(p);
#pragma unroll
    for (int i = 0; i < kMaxDPL; ++i) acc[i] *= corr;
    m = (mnew == kNegInf) ? m : mnew;
    psh[w][lane] = p;
    ish[w][lane] = src;
    __builtin_amdgcn_wave_barrier();
    const int nt = static_cast<int>(min<int64_t>(kTile, K - j0));
    for (int jj = 0; jj < nt; ++jj) {
      const int64_t s = ish[w][jj];
      if (s < 0) continue;  // uniform across the wave
      const float pj = psh[w][jj];
      const int64_t vbase = ((b * S + s) * 2 + 1) * D;
#pragma unroll
      for (int i = 0; i < kMaxDPL; ++i) {
        const int d = lane + 64 * i;
        if (d < D) acc[i] = fmaf(pj, ld<DT>(kv, vbase + d), acc[i]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  // sink joins the normaliser once: M = max(m, sink)
  const float M = fmaxf(m, sk);
  const float cm = (m == kNegInf) ? 0.0f : __expf(m - M);
  const float den = l * cm + __expf(sk - M);
  const float f = M == kNegInf ? 0.0f : cm / den;  // no valid source and sink -inf: 0
#pragma unroll
  for (int i = 0; i < kMaxDPL; ++i) {
    const int d = lane + 64 * i;
    if (d < D) st<DT>(out, row * D + d, acc[i] * f);
  }
}

// ------------------------------------------------------------------------------------------
// 2. quantised decode attention
// ------------------------------------------------------------------------------------------
struct QAttnArgs {
  const uint16_t* q;      // [B, H, D] bf16
  const uint8_t* codes;   // [B, S, D or D/2]
  const float* scale;     // [B, S]
  const int64_t* sel;     // [B, K] or null
  const uint16_t* win;    // [B, W, D] bf16
  const float* sink;      // [H]
  const float* diag;      // [D]
  int64_t S, K, W;
  int H, ts;              // ts: sources per tile
  int n_comp_tiles, n_tiles;
  float sm_scale, wscale;
  float* part;            // [B, n_tiles, H, D + 2]
  uint16_t* out;          // [B, H, D] bf16
};

__device__ __forceinline__ float round_bf16(float v) {
  return bf16_to_f32(pack_bf16x2(v, 0.0f) & 0xffffu);
}

// One workgroup = one tile of `ts` sources of one row, all heads.  Compressed sources are gathered
// by index and dequantised on load exactly as PolarQuant.decode(..., bf16) (the engine attends the
// bf16 dequantised cache, serving.py:346-376), window sources are the bf16 rows as stored.
template <int BITS, int D>
__global__ __launch_bounds__(kThreads) void quant_attn_partial_kernel(QAttnArgs a) {
  constexpr int EPL = D < 8 ? D : 8;
  constexpr int LPV = D / EPL;
  constexpr int VPW = 64 / LPV;
  constexpr int DP = D + 1;  // padded LDS row: conflict-free column walks
  extern __shared__ float smem[];
  const int H = a.H, ts = a.ts;
  float* qs = smem;         // H*D
  float* X = qs + H * D;    // ts*DP
  float* okf = X + ts * DP; // ts (1 = source present, 0 = skipped index)
  float* P = okf + ts;      // H*ts
  float* stat = P + H * ts; // 2H (tile max, tile sum)

  const int64_t b = blockIdx.y;
  const int tile = blockIdx.x;
  const bool comp = tile < a.n_comp_tiles;
  const int64_t n_src = comp ? a.K : a.W;  // (without sel: blocks 0 .. K-1 in order)
  const int64_t j0 = static_cast<int64_t>(comp ? tile : tile - a.n_comp_tiles) * ts;
  const int nt = static_cast<int>(min<int64_t>(ts, n_src - j0));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;

  for (int i = threadIdx.x; i < H * D; i += kThreads) qs[i] = bf16_to_f32(a.q[b * H * D + i]);

  if (comp) {
    constexpr int RB = BITS == 8 ? D : D / 2;
    const int sub = lane % LPV, slot = lane / LPV;
    float dg[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) dg[e] = a.diag[sub * EPL + e];
    for (int r0 = w * VPW; r0 < nt; r0 += (kThreads / 64) * VPW) {
      const int jj = r0 + slot;
      int64_t s = -1;
      if (jj < nt) s = a.sel ? a.sel[b * a.K + j0 + jj] : j0 + jj;
      const bool valid = jj < nt && s >= 0 && s < a.S;  // uniform within a lane group (one row)
      if (jj < nt) {
        // A skipped index still gets a zero row: the PV pass multiplies every staged row by its
        // (zero) probability, and 0 * stale LDS contents could be NaN.
        float v[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[e] = 0.0f;
        if (valid) decode_lane<BITS, D>(a.codes + (b * a.S + s) * RB, a.scale[b * a.S + s], sub, dg, a.wscale, v);
#pragma unroll
        for (int e = 0; e < EPL; ++e) X[jj * DP + sub * EPL + e] = round_bf16(v[e]);
        if (sub == 0) okf[jj] = valid ? 1.0f : 0.0f;
      }
    }
  } else {
    for (int e = threadIdx.x; e < nt * D; e += kThreads) {
      const int jj = e / D, d = e % D;
      X[jj * DP + d] = bf16_to_f32(a.win[(b * a.W + j0 + jj) * D + d]);
    }
    for (int jj = threadIdx.x; jj < nt; jj += kThreads) okf[jj] = 1.0f;
  }
  __syncthreads();

  // logits l = scale * q.K
  for (int p = threadIdx.x; p < H * nt; p += kThreads) {
    const int h = p / nt, jj = p % nt;
    const float* qh = qs + h * D;
    const float* xj = X + jj * DP;
    float dot = 0.0f;
#pragma unroll 8
    for (int d = 0; d < D; ++d) dot = fmaf(qh[d], xj[d], dot);
    P[h * ts + jj] = okf[jj] == 0.0f ? kNegInf : dot * a.sm_scale;
  }
  __syncthreads();

  // per-head tile softmax (one wave per head, round robin)
  for (int h = w; h < H; h += kThreads / 64) {
    float mx = kNegInf;
    for (int jj = lane; jj < nt; jj += 64) mx = fmaxf(mx, P[h * ts + jj]);
    mx = wave_max(mx);
    float sum = 0.0f;
    for (int jj = lane; jj < nt; jj += 64) {
      const float l = P[h * ts + jj];
      const float e = l == kNegInf ? 0.0f : __expf(l - mx);
      sum += e;
      P[h * ts + jj] = e;
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      stat[2 * h] = mx;
      stat[2 * h + 1] = sum;
    }
  }
  __syncthreads();

  // PV (K = V: the same staged rows)
  float* dst = a.part + ((b * a.n_tiles + tile) * H) * (D + 2);
  for (int p = threadIdx.x; p < H * D; p += kThreads) {
    const int h = p / D, d = p % D;
    const float* ph = P + h * ts;
    float acc = 0.0f;
    for (int jj = 0; jj < nt; ++jj) acc = fmaf(ph[jj], X[jj * DP + d], acc);
    dst[h * (D + 2) + 2 + d] = acc;
  }
  for (int h = threadIdx.x; h < H; h += kThreads) {
    dst[h * (D + 2)] = stat[2 * h];
    dst[h * (D + 2) + 1] = stat[2 * h + 1];
  }
}

// Merge the tiles of one row: M = max(sink, tile maxima), L = e^{sink-M} + sum_t e^{m_t-M} l_t,
// out = sum_t e^{m_t-M} acc_t / L  (the sink counted once, aether_pipeline/serving.py:125-129).
__global__ __launch_bounds__(kThreads) void quant_attn_combine_kernel(QAttnArgs a, int D) {
  extern __shared__ float smem[];
  const int H = a.H;
  float* fac = smem;                 // n_tiles * H
  float* den = fac + a.n_tiles * H;  // H
  const int64_t b = blockIdx.x;
  const float* part = a.part + (b * a.n_tiles) * H * (D + 2);
  for (int h = threadIdx.x; h < H; h += kThreads) {
    const float sk = a.sink[h];
    float M = sk;
    for (int t = 0; t < a.n_tiles; ++t) M = fmaxf(M, part[(t * H + h) * (D + 2)]);
    float L = __expf(sk - M);
    for (int t = 0; t < a.n_tiles; ++t) {
      const float mt = part[(t * H + h) * (D + 2)];
      const float f = mt == kNegInf ? 0.0f : __expf(mt - M);
      fac[t * H + h] = f;
      L += f * part[(t * H + h) * (D + 2) + 1];
    }
    den[h] = M == kNegInf ? 1.0f : L;  // no source and sink -inf: every factor is 0, so 0
  }
  __syncthreads();
  for (int p = threadIdx.x; p < H * D; p += kThreads) {
    const int h = p / D, d = p % D;
    float o = 0.0f;
    for (int t = 0; t < a.n_tiles; ++t) o = fmaf(fac[t * H + h], part[(t * H + h) * (D + 2) + 2 + d], o);
    a.out[b * H * D + p] = static_cast<uint16_t>(pack_bf16x2(o / den[h], 0.0f) & 0xffffu);
  }
}

typedef void (*qattn_fn)(QAttnArgs);

template <int BITS>
qattn_fn pick_qattn(int D) {
  switch (D) {
    case 2: return quant_attn_partial_kernel<BITS, 2>;
    case 4: return quant_attn_partial_kernel<BITS, 4>;
    case 8: return quant_attn_partial_kernel<BITS, 8>;
    case 16: return quant_attn_partial_kernel<BITS, 16>;
    case 32: return quant_attn_partial_kernel<BITS, 32>;
    case 64: return quant_attn_partial_kernel<BITS, 64>;
    case 128: return quant_attn_partial_kernel<BITS, 128>;
    case 256: return quant_attn_partial_kernel<BITS, 256>;
    default: return nullptr;
  }
}

// ------------------------------------------------------------------------------------------
// 3. hca_compress
// ------------------------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(kThreads) void hca_compress_kernel(const void* __restrict__ c, const void* __restrict__ z,
                                                                int64_t B, int64_t M, int64_t D, void* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= B * D) return;
  const int64_t b = i / D, d = i % D;
  float mx = kNegInf;
  for (int64_t m = 0; m < M; ++m) mx = fmaxf(mx, ld<DT>(z, (b * M + m) * D + d));
  float den = 0.0f, acc = 0.0f;
  for (int64_t m = 0; m < M; ++m) {
    const float e = __expf(ld<DT>(z, (b * M + m) * D + d) - mx);
    den += e;
    acc = fmaf(e, ld<DT>(c, (b * M + m) * D + d), acc);
  }
  st<DT>(out, i, acc / den);
}

__global__ void zero_u16_kernel(uint16_t* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Dynamic LDS above 64 KB must be enabled per kernel; the attribute is set on every launch path
// (idempotent and cheap).
void allow_big_lds(const void* fn) {
  static std::mutex mu;
  static std::unordered_set<const void*> done;
  std::lock_guard<std::mutex> lock(mu);
  if (done.insert(fn).second) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}

template <int DT>
int launch_sparse(int idx_kind, const void* q, const void* kv, const void* topk, const void* sink, int scalar,
                  int64_t B, int64_t T, int64_t H, int64_t D, int64_t S, int64_t K, float scale, void* out,
                  hipStream_t st) {
  const int64_t rows = B * T * H;
  const dim3 grid(static_cast<uint32_t>(ceil_div(rows, kThreads / 64)));
  if (idx_kind == 0)
    hipLaunchKernelGGL((sparse_attn_kernel<DT, 0>), grid, dim3(kThreads), 0, st, q, kv, topk, sink, scalar, rows, T, H,
                       static_cast<int>(D), S, K, scale, out);
  else if (idx_kind == 4)
    hipLaunchKernelGGL((sparse_attn_kernel<DT, 4>), grid, dim3(kThreads), 0, st, q, kv, topk, sink, scalar, rows, T, H,
                       static_cast<int>(D), S, K, scale, out);
  else
    hipLaunchKernelGGL((sparse_attn_kernel<DT, 8>), grid, dim3(kThreads), 0, st, q, kv, topk, sink, scalar, rows, T, H,
                       static_cast<int>(D), S, K, scale, out);
  return AEKV_OK;
}

int sparse_common(const void* q, const void* kv, const void* topk, int idx_kind, const void* sink, int64_t sink_numel,
                  int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t D, int64_t S, int64_t K, float scale,
                  void* ws, size_t ws_bytes, void* out, void* stream, const char* who) {
  if (!is_float_dtype(dtype)) return fail(AEKV_ERR_DTYPE, "%s: dtype %d is not f32/f16/bf16", who, dtype);
  if (B < 0 || T < 0 || H < 0 || D < 0 || S < 0 || K < 0) return fail(AEKV_ERR_SHAPE, "%s: negative size", who);
  if (D > kMaxD) return fail(AEKV_ERR_UNSUPPORTED, "%s: head_dim %lld exceeds %d", who, (long long)D, kMaxD);
  if (sink_numel != 1 && sink_numel != H)
    return fail(AEKV_ERR_SHAPE, "sink must be a scalar or a [num_heads] tensor");
  const int64_t rows = B * T * H;
  if (rows == 0 || D == 0) return AEKV_OK;
  if (ceil_div(rows, kThreads / 64) > 0x7fffffffLL) return fail(AEKV_ERR_UNSUPPORTED, "%s: too many rows", who);
  if (!q || !sink || !out || (K > 0 && (!kv || (idx_kind != 0 && !topk))))
    return fail(AEKV_ERR_VALUE, "%s: null pointer", who);
  const hipStream_t st = as_stream(stream);
  const int scalar = sink_numel == 1 ? 1 : 0;
  if (sink_attention_mfma_supported(dtype, D) && is_aligned(q, 16) && is_aligned(out, 8) &&
      (K == 0 || is_aligned(kv, 16)) && is_aligned(sink, 2))
    return sink_attention_mfma(q, kv, topk, idx_kind, sink, scalar, dtype, B, T, H, S, K, scale, ws, ws_bytes, out, st,
                               who);
  if (dtype == AEKV_F32) launch_sparse<AEKV_F32>(idx_kind, q, kv, topk, sink, scalar, B, T, H, D, S, K, scale, out, st);
  else if (dtype == AEKV_F16) launch_sparse<AEKV_F16>(idx_kind, q, kv, topk, sink, scalar, B, T, H, D, S, K, scale, out, st);
  else launch_sparse<AEKV_BF16>(idx_kind, q, kv, topk, sink, scalar, B, T, H, D, S, K, scale, out, st);
  return check_launch(who);
}

struct QLayout {
  int ts, n_comp_tiles, n_tiles;
  size_t part_bytes;
};

QLayout qlayout(int64_t B, int64_t H, int64_t D, int64_t n_comp, int64_t W) {
  QLayout l;
  int ts = static_cast<int>(kTileFloats / (D > 0 ? D : 1));
  if (ts > 256) ts = 256;
  if (ts < 1) ts = 1;
  l.ts = ts;
  l.n_comp_tiles = static_cast<int>(ceil_div(n_comp, ts));
  l.n_tiles = l.n_comp_tiles + static_cast<int>(ceil_div(W, ts));
  l.part_bytes = align_up(static_cast<size_t>(B) * l.n_tiles * H * (D + 2) * 4, 256);
  return l;
}

}  // namespace
}  // namespace aekv

using namespace aekv;

extern "C" int aekv_sparse_sink_attention_ws(const void* q, const void* kv, const void* topk, int32_t idx_dtype,
                                             const void* sink, int64_t sink_numel, int32_t dtype, int64_t B,
                                             int64_t T, int64_t H, int64_t D, int64_t S, int64_t K,
                                             float softmax_scale, void* ws, size_t ws_bytes, void* out,
                                             void* stream) {
  if (idx_dtype != AEKV_I32 && idx_dtype != AEKV_I64) return fail(AEKV_ERR_DTYPE, "topk_indices must be int32 or int64");
  return sparse_common(q, kv, topk, idx_dtype == AEKV_I32 ? 4 : 8, sink, sink_numel, dtype, B, T, H, D, S, K,
                       softmax_scale, ws, ws_bytes, out, stream, "aekv_sparse_sink_attention");
}

extern "C" int aekv_sparse_sink_attention(const void* q, const void* kv, const void* topk, int32_t idx_dtype,
                                          const void* sink, int64_t sink_numel, int32_t dtype, int64_t B, int64_t T,
                                          int64_t H, int64_t D, int64_t S, int64_t K, float softmax_scale, void* out,
                                          void* stream) {
  return aekv_sparse_sink_attention_ws(q, kv, topk, idx_dtype, sink, sink_numel, dtype, B, T, H, D, S, K,
                                       softmax_scale, nullptr, 0, out, stream);
}

extern "C" int aekv_tiled_prefill_attention_ws(const void* q, const void* kv, const void* sink, int64_t sink_numel,
                                               int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t D, int64_t S,
                                               float softmax_scale, int32_t tile_size, void* ws, size_t ws_bytes,
                                               void* out, void* stream) {
  if (tile_size <= 0) return fail(AEKV_ERR_VALUE, "tile_size must be positive");
  return sparse_common(q, kv, nullptr, 0, sink, sink_numel, dtype, B, T, H, D, S, S, softmax_scale, ws, ws_bytes, out,
                       stream, "aekv_tiled_prefill_attention");
}

extern "C" int aekv_tiled_prefill_attention(const void* q, const void* kv, const void* sink, int64_t sink_numel,
                                            int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t D, int64_t S,
                                            float softmax_scale, int32_t tile_size, void* out, void* stream) {
  return aekv_tiled_prefill_attention_ws(q, kv, sink, sink_numel, dtype, B, T, H, D, S, softmax_scale, tile_size,
                                         nullptr, 0, out, stream);
}

extern "C" size_t aekv_sink_attention_workspace_size(int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t D,
                                                     int64_t S, int64_t K) {
  if (!sink_attention_mfma_supported(dtype, D) || B <= 0 || T <= 0 || H <= 0 || S < 0) return 0;
  return K < 0 ? sink_attention_mfma_workspace(true, B, T, H, S, S) : sink_attention_mfma_workspace(false, B, T, H, S, K);
}

extern "C" size_t aekv_quant_attention_workspace_size(int64_t B, int64_t H, int64_t D, int64_t n_comp, int64_t W) {
  if (B <= 0 || H <= 0 || D <= 0) return 256;
  return qlayout(B, H, D, n_comp, W).part_bytes;
}

extern "C" int aekv_quant_sink_attention(const void* q, const void* codes, const float* scale, const int64_t* sel,
                                         const void* window, const float* sink, const float* diag, int64_t B, int64_t H,
                                         int64_t D, int64_t S, int64_t n_sel, int64_t W, int32_t bits, float softmax_scale,
                                         void* ws, size_t ws_bytes, void* out, void* stream) {
  const char* who = "aekv_quant_sink_attention";
  if (bits != 4 && bits != 8) return fail(AEKV_ERR_VALUE, "bits must be 4 or 8, got %d", bits);
  if (!is_pow2(D)) return fail(AEKV_ERR_VALUE, "WHT requires last dim to be a power of 2, got %lld", (long long)D);
  if (D < 2 || D > 256) return fail(AEKV_ERR_UNSUPPORTED, "%s: head_dim %lld outside [2, 256]", who, (long long)D);
  if (B < 0 || H <= 0 || S < 0 || W < 0) return fail(AEKV_ERR_SHAPE, "%s: bad sizes", who);
  if (H * D > 4096) return fail(AEKV_ERR_UNSUPPORTED, "%s: H*D=%lld exceeds 4096", who, (long long)(H * D));
  if (B > 65535) return fail(AEKV_ERR_UNSUPPORTED, "%s: B exceeds 65535", who);
  // in order: every block (n_sel < 0, HCA) or, without sel, the first n_sel blocks of each row
  const bool all_blocks = n_sel < 0 || !sel;
  const int64_t K = all_blocks ? 0 : n_sel;
  const int64_t n_comp = n_sel < 0 ? S : (all_blocks ? std::min(n_sel, S) : K);
  const QLayout l = qlayout(B, H, D, n_comp, W);
  if (B == 0) return AEKV_OK;
  if (!q || !sink || !diag || !out || (n_comp > 0 && (!codes || !scale)) || (W > 0 && !window))
    return fail(AEKV_ERR_VALUE, "%s: null pointer", who);
  if (l.n_tiles == 0) {
    // no sources: every weight is zero -> out = 0 (serving.py:451-452)
    const int64_t n16 = B * H * D;
    hipLaunchKernelGGL(zero_u16_kernel, dim3(static_cast<uint32_t>(ceil_div(n16, kThreads))), dim3(kThreads), 0,
                       as_stream(stream), static_cast<uint16_t*>(out), n16);
    return check_launch(who);
  }
  if (!ws || ws_bytes < l.part_bytes)
    return fail(AEKV_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who, l.part_bytes, ws_bytes);
  if (quant_attn_mfma_supported(H, D) && quant_attn_mfma_fits(B, n_comp + W) && use_specialised_codec() &&
      is_aligned(q, 16) && is_aligned(out, 8) && is_aligned(ws, 16) &&
      is_aligned(diag, 16) && (n_comp == 0 || is_aligned(codes, 16)) && (W == 0 || is_aligned(window, 16)))
    return launch_quant_attn_mfma(q, codes, scale, sel, window, sink, diag, B, H, S, all_blocks ? n_comp : K,
                                  all_blocks, W, bits, softmax_scale, ws, out, as_stream(stream), who);
  if (l.n_tiles > 65535) return fail(AEKV_ERR_UNSUPPORTED, "%s: too many source tiles", who);
  QAttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.codes = static_cast<const uint8_t*>(codes);
  a.scale = scale;
  a.sel = all_blocks ? nullptr : sel;
  a.win = static_cast<const uint16_t*>(window);
  a.sink = sink;
  a.diag = diag;
  a.S = S;
  a.K = all_blocks ? n_comp : K;
  a.W = W;
  a.H = static_cast<int>(H);
  a.ts = l.ts;
  a.n_comp_tiles = l.n_comp_tiles;
  a.n_tiles = l.n_tiles;
  a.sm_scale = softmax_scale;
  a.wscale = wht_scale(static_cast<int>(D));
  a.part = static_cast<float*>(ws);
  a.out = static_cast<uint16_t*>(out);
  const hipStream_t st = as_stream(stream);
  qattn_fn fn = bits == 8 ? pick_qattn<8>(static_cast<int>(D)) : pick_qattn<4>(static_cast<int>(D));
  allow_big_lds(reinterpret_cast<const void*>(fn));
  const size_t sm1 = sizeof(float) * (H * D + static_cast<size_t>(l.ts) * (D + 1) + l.ts + H * l.ts + 2 * H);
  if (sm1 > 160 * 1024) return fail(AEKV_ERR_UNSUPPORTED, "%s: source tile does not fit in LDS", who);
  hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(l.n_tiles), static_cast<uint32_t>(B)), dim3(kThreads), sm1, st, a);
  if (int rc = check_launch(who)) return rc;
  const size_t sm2 = sizeof(float) * (static_cast<size_t>(l.n_tiles) * H + H);
  if (sm2 > 160 * 1024) return fail(AEKV_ERR_UNSUPPORTED, "%s: too many tiles for the combine", who);
  allow_big_lds(reinterpret_cast<const void*>(quant_attn_combine_kernel));
  hipLaunchKernelGGL(quant_attn_combine_kernel, dim3(static_cast<uint32_t>(B)), dim3(kThreads), sm2, st, a,
                     static_cast<int>(D));
  return check_launch(who);
}

extern "C" size_t aekv_quant_prefill_workspace_size(int64_t B, int64_t T, int64_t H, int64_t n_comp, int64_t Wt) {
  if (B <= 0 || T <= 0 || H <= 0) return 256;
  const int64_t nc = std::max<int64_t>(n_comp, 0);
  // per-target split partials (CSA) or every block decoded to bf16 (HCA: n_comp = S)
  const size_t rows = quant_attn_mfma_workspace(B * T, H, nc + std::max<int64_t>(Wt, 0));
  const size_t blocks = hca_prefill_flash_workspace(B, nc);
  return std::max<size_t>(256, std::max(rows, blocks));
}

extern "C" int aekv_quant_prefill_attention(const void* q, const void* codes, const float* scale, const int64_t* sel,
                                            const int32_t* visible, const void* window, const int32_t* win_start,
                                            const int32_t* win_len, const float* sink, const float* diag, int64_t B,
                                            int64_t T, int64_t H, int64_t D, int64_t S, int64_t n_sel, int64_t Wt,
                                            int32_t bits, float softmax_scale, void* ws, size_t ws_bytes, void* out,
                                            void* stream) {
  const char* who = "aekv_quant_prefill_attention";
  if (bits != 4 && bits != 8) return fail(AEKV_ERR_VALUE, "bits must be 4 or 8, got %d", bits);
  if (!quant_attn_mfma_supported(H, D))
    return fail(AEKV_ERR_UNSUPPORTED, "%s: head_dim %lld with %lld heads (128 and at most 16 supported)", who,
                (long long)D, (long long)H);
  if (B > 0 && !quant_attn_mfma_fits(B * T, (n_sel < 0 ? S : n_sel) + Wt))
    return fail(AEKV_ERR_UNSUPPORTED, "%s: %lld targets with %lld sources exceed the launch limits", who,
                (long long)(B * T), (long long)((n_sel < 0 ? S : n_sel) + Wt));
  if (B < 0 || T < 1 || S < 0 || Wt < 0) return fail(AEKV_ERR_SHAPE, "%s: bad sizes", who);
  if (B > 0 && T > 65535 / B) return fail(AEKV_ERR_UNSUPPORTED, "%s: B*T exceeds 65535", who);
  const bool all_blocks = n_sel < 0;  // HCA: blocks 0 .. visible-1 in order
  const int64_t K = all_blocks ? 0 : n_sel;
  const int64_t n_comp = all_blocks ? S : K;
  if (B == 0) return AEKV_OK;
  if (!q || !sink || !diag || !out || (n_comp > 0 && (!codes || !scale)) || (Wt > 0 && !window) || (K > 0 && !sel))
    return fail(AEKV_ERR_VALUE, "%s: null pointer", who);
  if (!is_aligned(q, 16) || !is_aligned(out, 8) || !is_aligned(diag, 16) || (n_comp > 0 && !is_aligned(codes, 16)) ||
      (Wt > 0 && !is_aligned(window, 16)) || !is_aligned(sink, 4) || (scale && !is_aligned(scale, 4)))
    return fail(AEKV_ERR_ALIGN, "%s: misaligned pointer", who);
  if (all_blocks && hca_prefill_flash_supported(H, D)) {
    // HCA: decode every block once (exactly PolarQuant.decode's bf16 values) into the workspace,
    // then the flash kernel over [blocks; window] with per-target masks
    const size_t need = S > 0 ? hca_prefill_flash_workspace(B, S) : 0;
    if (need > 0 && (!ws || ws_bytes < need))
      return fail(AEKV_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who, need, ws_bytes);
    if (need > 0 && !is_aligned(ws, 256)) return fail(AEKV_ERR_ALIGN, "%s: workspace must be 256-byte aligned", who);
    if (S > 0) {
      if (int rc = aekv_tq_decode(codes, scale, B * S, 128, bits, diag, ws, AEKV_BF16, stream)) return rc;
    }
    return launch_hca_prefill_flash(q, ws, window, visible, win_start, win_len, sink, B, T, H, S, Wt,
                                    softmax_scale, out, as_stream(stream), who);
  }
  const size_t need = quant_attn_mfma_workspace(B * T, H, n_comp + Wt);
  if (need > 0 && (!ws || ws_bytes < need))
    return fail(AEKV_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who, need, ws_bytes);
  // without per-target window slices every target sees the whole [0, Wt) window
  return launch_quant_attn_mfma_rows(q, codes, scale, sel, visible, window, win_start, win_len, sink, diag, B * T, T,
                                     H, S, n_comp, all_blocks, Wt, bits, softmax_scale, ws, out, as_stream(stream),
                                     who);
}

extern "C" int aekv_hca_compress(const void* c, const void* z, int32_t dtype, int64_t B, int64_t M, int64_t D, void* out,
                                 void* stream) {
  const char* who = "aekv_hca_compress";
  if (!is_float_dtype(dtype)) return fail(AEKV_ERR_DTYPE, "%s: dtype %d is not f32/f16/bf16", who, dtype);
  if (B < 0 || M < 0 || D < 0) return fail(AEKV_ERR_SHAPE, "%s: negative size", who);
  if (B * D == 0) return AEKV_OK;
  if (M == 0) return fail(AEKV_ERR_SHAPE, "%s: empty compression window", who);
  if (!c || !z || !out) return fail(AEKV_ERR_VALUE, "%s: null pointer", who);
  const dim3 grid(static_cast<uint32_t>(ceil_div(B * D, kThreads)));
  const hipStream_t st = as_stream(stream);
  if (dtype == AEKV_F32) hipLaunchKernelGGL(hca_compress_kernel<AEKV_F32>, grid, dim3(kThreads), 0, st, c, z, B, M, D, out);
  else if (dtype == AEKV_F16) hipLaunchKernelGGL(hca_compress_kernel<AEKV_F16>, grid, dim3(kThreads), 0, st, c, z, B, M, D, out);
  else hipLaunchKernelGGL(hca_compress_kernel<AEKV_BF16>, grid, dim3(kThreads), 0, st, c, z, B, M, D, out);
  return check_launch(who);
}
