// Drop-in sink attention on the matrix cores, head_dim 128, bf16 or fp16.
//
// Reference: sparse_sink_attention (aether_kernels/sparse_attention.py:8-16; semantics
// aether_kernels/csrc/sparse_sink_attention_cuda.cu:47-114 and the torch backend
// aether_pipeline/serving.py:99-130) and tiled_prefill_attention (aether_kernels/sparse_attention.py:
// 19-42) with the sink counted once in the normaliser (aether_2b/modeling.py:158-178).
//
// gather_attn_kernel: one workgroup per (target, group of 16 heads).  Every head of a target
// attends the same sources (its K indices, or every source for the dense call), so the heads are
// the 16 columns of v_mfma_f32_16x16x32_{bf16,f16} and the sources stream through the waves in
// groups of 32 (two blocks of 16), straight from global memory into registers:
//   S^T = K Q^T   A = key rows (lane = key, 8 consecutive dims per lane group and k-step),
//                 B = the target's queries (lane = head); each lane then owns head lane & 15.
//   online softmax of the lane's head over the group;
//   V^T           the V rows times a 0/1 column selector (exact), which lands them in the A layout
//                 of O^T += V^T P^T; B = P^T comes straight from the softmax registers.
// The waves' (max, sum, O) are merged through LDS at the end, where the sink joins once.  A
// target with many sources and a launch with few targets split the sources over several
// workgroups (grid z); each writes its unnormalised (max, sum, O) per head and
// sink_attn_combine_kernel merges the pieces with the sink (the same merge, across workgroups).
// Weights are exponentials in base 2 of log2(e)-scaled logits, in both kernels and the pieces.
//
// The weights enter the products rounded to the input type, and the normaliser sums those
// rounded weights, so the output is an exact convex combination of the V rows with weights whose
// ratios carry one rounding each (2^-9 relative in bf16, 2^-12 in fp16).
#include <algorithm>

#include "aekv_common.h"

namespace aekv {
namespace {

constexpr int kD = 128;
constexpr int kGroup = 32;            // sources per wave step
constexpr int kObStride = kD + 4;     // merge rows: head h at bank 4h (no conflicts)
constexpr int kPartStride = kD + 4;   // one piece of one (target, head): max, sum, 2 pad, O[128]
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;

// The matrix instruction, rounding and constants of one input type.
template <int DT>
struct Elem;
template <>
struct Elem<AEKV_BF16> {
  typedef bf16x8_t v8;
  static constexpr uint32_t kOnePair = 0x3F803F80u;
  __device__ static f32x4_t mma(v8 a, v8 b, f32x4_t c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
  __device__ static uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
  __device__ static float to_f32(uint32_t bits) { return bf16_to_f32(bits); }
};
template <>
struct Elem<AEKV_F16> {
  typedef f16x8_t v8;
  static constexpr uint32_t kOnePair = 0x3C003C00u;
  __device__ static f32x4_t mma(v8 a, v8 b, f32x4_t c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
  __device__ static uint32_t pack(float lo, float hi) { return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16); }
  __device__ static float to_f32(uint32_t bits) { return f16_to_f32(bits); }
};

struct GatherArgs {
  const uint16_t* q;     // [B, T, H, 128]
  const uint16_t* kv;    // [B, S, 2, 128]: K then V of each source
  const void* idx;       // [B, T, K] int32 / int64 (null: dense, source j = j)
  const uint16_t* sink;  // [H] or [1]
  int sink_scalar;
  int H;
  int64_t T, S, K;       // K: sources per target (S for the dense call)
  float scale2;          // softmax scale * log2(e)
  int n_split;           // source pieces per target (grid z)
  int64_t gps;           // 32-source groups per piece
  float* part;           // [B * T * H, n_split, kPartStride] when n_split > 1
  uint16_t* out;         // [B, T, H, 128]
};

template <int NW>
struct GatherLds {
  float ob[NW * 16 * kObStride];  // [wave][head][dims]
  float st[NW * 16 * 2];          // [wave][head][max, sum]
  float inv[16];                  // [head] 1 / normaliser
};

// IDX: 0 dense, 4 int32 indices, 8 int64 indices.  NW waves per workgroup.
template <int DT, int IDX, int NW>
__global__ __launch_bounds__(64 * NW) void gather_attn_kernel(GatherArgs a) {
  using E = Elem<DT>;
  using v8 = typename E::v8;
  __shared__ __align__(16) GatherLds<NW> L;  // 16-byte aligned: the merge uses 16-byte accesses
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  const int64_t bt = blockIdx.x;  // b * T + t
  const int h0 = 16 * static_cast<int>(blockIdx.y);
  const int nh = min(16, a.H - h0);
  const int64_t b = static_cast<uint32_t>(bt) / static_cast<uint32_t>(a.T);  // (32-bit: bt < 2^31, 1 <= T)
  const int64_t K = a.K, S = a.S;

  // the target's queries as the B operand: lane (head c16), k-step ks = dims 32 ks + 8 g .. + 7
  v8 qb[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (c16 < nh) v = *reinterpret_cast<const uint4*>(a.q + (bt * a.H + h0 + c16) * kD + 32 * ks + 8 * g);
    qb[ks] = __builtin_bit_cast(v8, v);
  }
  // 0/1 selectors: column c16 of esel[hv] picks dim 32 ks + 16 hv + c16 of k-step ks, i.e. element
  // c16 & 7 of lane group 2 hv + (c16 >> 3)
  v8 esel[2];
#pragma unroll
  for (int hv = 0; hv < 2; ++hv) {
    uint32_t w[4];
    const bool mine = g == 2 * hv + (c16 >> 3);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j0 = 2 * e;
      w[e] = (mine && (c16 & 7) == j0 ? (E::kOnePair & 0xFFFFu) : 0u) |
             (mine && (c16 & 7) == j0 + 1 ? (E::kOnePair & 0xFFFF0000u) : 0u);
    }
    esel[hv] = __builtin_bit_cast(v8, make_uint4(w[0], w[1], w[2], w[3]));
  }

  const uint16_t* kvb = a.kv + b * S * (2 * kD);
  float m_run = kNegInf, l_run = 0.0f;
  f32x4_t O[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) O[nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const int split = blockIdx.z;
  const int64_t g_end = min((K + kGroup - 1) / kGroup, (split + 1) * a.gps);
#pragma unroll 1
  for (int64_t G = split * a.gps + wv; G < g_end; G += NW) {
    // lane (key c16 of block kb): its source's K and V rows (both blocks requested before use)
    bool ok[2];
    uint4 kr[2][4], vr[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int64_t j = G * kGroup + 16 * kb + c16;
      int64_t src = -1;
      if (j < K) {
        if constexpr (IDX == 0) src = j;
        else if constexpr (IDX == 4) src = static_cast<const int32_t*>(a.idx)[bt * K + j];
        else src = static_cast<const int64_t*>(a.idx)[bt * K + j];
      }
      ok[kb] = src >= 0 && src < S;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        kr[kb][ks] = make_uint4(0u, 0u, 0u, 0u);
        vr[kb][ks] = make_uint4(0u, 0u, 0u, 0u);
      }
      if (ok[kb]) {
        const uint16_t* row = kvb + src * (2 * kD) + 8 * g;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          kr[kb][ks] = *reinterpret_cast<const uint4*>(row + 32 * ks);
          vr[kb][ks] = *reinterpret_cast<const uint4*>(row + kD + 32 * ks);
        }
      }
    }
    // st[kb][i] = S[head c16][key 16 kb + 4 g + i of the group]
    f32x4_t st[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      st[kb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) st[kb] = E::mma(__builtin_bit_cast(v8, kr[kb][ks]), qb[ks], st[kb]);
    }
    uint32_t pw[4];  // the weights as packed pairs, element 4 kb + i <-> key 16 kb + 4 g + i
    {
      float lg[2][4];
      float tm = kNegInf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        // ok[kb] belongs to key c16, so bit 4 g + i of its ballot is the validity of key 4 g + i
        const uint64_t okm = __builtin_amdgcn_ballot_w64(ok[kb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lg[kb][i] = ((okm >> (4 * g + i)) & 1u) ? st[kb][i] * a.scale2 : kNegInf;
          tm = fmaxf(tm, lg[kb][i]);
        }
      }
      tm = fmaxf(tm, xor_lane<16>(tm));
      tm = fmaxf(tm, xor_lane<32>(tm));
      const float mnew = fmaxf(m_run, tm);
      const float corr = m_run == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m_run - mnew);
      float ps = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          const float p0 = lg[kb][i] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(lg[kb][i] - mnew);
          const float p1 = lg[kb][i + 1] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(lg[kb][i + 1] - mnew);
          const uint32_t w = E::pack(p0, p1);
          pw[2 * kb + i / 2] = w;
          ps += E::to_f32(w & 0xFFFFu) + E::to_f32(w >> 16);  // the weights as rounded
        }
      ps += xor_lane<16>(ps);
      ps += xor_lane<32>(ps);
      l_run = l_run * corr + ps;
      m_run = mnew;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) O[nb] *= corr;
    }
    const v8 pb = __builtin_bit_cast(v8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      // V columns 16 nb .. + 15 of the 32 keys: the V rows times the selector (exact)
      const f32x4_t v0 = E::mma(__builtin_bit_cast(v8, vr[0][nb >> 1]), esel[nb & 1], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
      const f32x4_t v1 = E::mma(__builtin_bit_cast(v8, vr[1][nb >> 1]), esel[nb & 1], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
      // A = V^T: lane (dim 16 nb + c16), element 4 kb + i <-> key 16 kb + 4 g + i (the order of pb)
      const v8 va = __builtin_bit_cast(
          v8, make_uint4(E::pack(v0[0], v0[1]), E::pack(v0[2], v0[3]), E::pack(v1[0], v1[1]), E::pack(v1[2], v1[3])));
      // O^T[nb][i] = O[head c16][dim 16 nb + 4 g + i]
      O[nb] = E::mma(va, pb, O[nb]);
    }
  }

  // ---- merge the waves; the sink joins the normaliser once (in the combine for a split) ----
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
    *reinterpret_cast<f32x4_t*>(L.ob + (wv * 16 + c16) * kObStride + 16 * nb + 4 * g) = O[nb];
  if (g == 0) {
    L.st[(wv * 16 + c16) * 2] = m_run;
    L.st[(wv * 16 + c16) * 2 + 1] = l_run;
  }
  __syncthreads();
  const bool whole = a.n_split == 1;
  if (threadIdx.x < nh) {
    const int h = threadIdx.x;
    const float sk = whole ? E::to_f32(a.sink[a.sink_scalar ? 0 : h0 + h]) * kLog2e : kNegInf;
    float M = sk;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, L.st[(w * 16 + h) * 2]);
    float den = whole ? __builtin_amdgcn_exp2f(sk - M) : 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float mw = L.st[(w * 16 + h) * 2];
      const float f = mw == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      den = fmaf(f, L.st[(w * 16 + h) * 2 + 1], den);
      L.st[(w * 16 + h) * 2] = f;
    }
    if (whole) {
      // no valid source and sink -inf: 0, as the reference kernel (its sum skips every index)
      L.inv[h] = M == kNegInf ? 0.0f : 1.0f / den;
    } else {
      float* dst = a.part + ((bt * a.H + h0 + h) * a.n_split + split) * kPartStride;
      dst[0] = M;
      dst[1] = den;
    }
  }
  __syncthreads();
  for (int p = threadIdx.x; p < nh * (kD / 4); p += 64 * NW) {
    const int h = p / (kD / 4), d4 = 4 * (p % (kD / 4));
    f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = L.st[(w * 16 + h) * 2];
      const f32x4_t o = *reinterpret_cast<const f32x4_t*>(L.ob + (w * 16 + h) * kObStride + d4);
      acc = f32x4_t{fmaf(f, o[0], acc[0]), fmaf(f, o[1], acc[1]), fmaf(f, o[2], acc[2]), fmaf(f, o[3], acc[3])};
    }
    if (whole) {
      const float r = L.inv[h];
      *reinterpret_cast<uint2*>(a.out + (bt * a.H + h0 + h) * kD + d4) =
          make_uint2(E::pack(acc[0] * r, acc[1] * r), E::pack(acc[2] * r, acc[3] * r));
    } else {
      *reinterpret_cast<f32x4_t*>(a.part + ((bt * a.H + h0 + h) * a.n_split + split) * kPartStride + 4 + d4) = acc;
    }
  }
}

// Merges the source pieces of each (target, head) row: M = max(sink, piece maxima),
// L = 2^(sink - M) + sum_p 2^(m_p - M) l_p, out = sum_p 2^(m_p - M) O_p / L (log2 units), as an
// online merge over chunks of 8 pieces whose loads are all issued together.  32 threads per row,
// 4 dims each, NT / 32 rows per workgroup: 8, or 2 when 8 would leave CUs without a workgroup, so
// that a call of few rows spreads its loads over as many CUs.
template <int DT, int NT>
__global__ __launch_bounds__(NT) void sink_attn_combine_kernel(const float* __restrict__ part, int n_split,
                                                               const uint16_t* __restrict__ sink, int sink_scalar,
                                                               int H, int rows, uint16_t* __restrict__ out) {
  using E = Elem<DT>;
  constexpr int kChunk = 8;
  const int row = static_cast<int>(blockIdx.x) * (NT / 32) + (static_cast<int>(threadIdx.x) >> 5);
  if (row >= rows) return;
  const int j = threadIdx.x & 31;
  const float* p = part + static_cast<int64_t>(row) * n_split * kPartStride;
  float m[kChunk], l[kChunk];
  f32x4_t o[kChunk];
  // A chunk's loads (and the sink's, with the first) all precede the empty asm that takes their
  // values, so every load is issued before the first wait (the compiler would otherwise wait for
  // the sink first, and move loads into the branches that use them, each with its own wait).  A
  // piece past n_split reads piece 0 and is replaced by the empty state.
  auto load_chunk = [&](const int s0, uint32_t* skb) {
    float2 ml[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const float* ps = p + (s0 + i < n_split ? s0 + i : 0) * kPartStride;
      ml[i] = *reinterpret_cast<const float2*>(ps);
      o[i] = *reinterpret_cast<const f32x4_t*>(ps + 4 + 4 * j);
    }
    if (skb) *skb = sink[sink_scalar ? 0 : row % H];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) asm volatile("" : "+v"(ml[i].x), "+v"(ml[i].y), "+v"(o[i]));
    if (skb) asm volatile("" : "+v"(*skb));
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const bool in = s0 + i < n_split;
      m[i] = in ? ml[i].x : kNegInf;
      l[i] = in ? ml[i].y : 0.0f;
      o[i] = in ? o[i] : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  uint32_t skb;
  load_chunk(0, &skb);
  const float sk = E::to_f32(skb) * kLog2e;
  float M = sk, den = sk == kNegInf ? 0.0f : 1.0f;
  f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < n_split; s0 += kChunk) {
    if (s0 > 0) load_chunk(s0, nullptr);
    float cm = M;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) cm = fmaxf(cm, m[i]);
    if (cm == kNegInf) continue;  // nothing yet (no sink, no source)
    const float r = M == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(M - cm);
    den *= r;
    acc *= r;
    M = cm;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const float f = m[i] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m[i] - M);
      den = fmaf(f, l[i], den);
      acc = f32x4_t{fmaf(f, o[i][0], acc[0]), fmaf(f, o[i][1], acc[1]), fmaf(f, o[i][2], acc[2]), fmaf(f, o[i][3], acc[3])};
    }
  }
  const float r = den > 0.0f ? 1.0f / den : 0.0f;
  *reinterpret_cast<uint2*>(out + static_cast<int64_t>(row) * kD + 4 * j) =
      make_uint2(E::pack(acc[0] * r, acc[1] * r), E::pack(acc[2] * r, acc[3] * r));
}

template <int DT, int IDX>
void launch_gather_t(const GatherArgs& a, int64_t rows, int hgroups, int nw, hipStream_t st) {
  const dim3 grid(static_cast<uint32_t>(rows), static_cast<uint32_t>(hgroups), static_cast<uint32_t>(a.n_split));
  if (nw == 8) hipLaunchKernelGGL((gather_attn_kernel<DT, IDX, 8>), grid, dim3(512), 0, st, a);
  else if (nw == 4) hipLaunchKernelGGL((gather_attn_kernel<DT, IDX, 4>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((gather_attn_kernel<DT, IDX, 2>), grid, dim3(128), 0, st, a);
}

// How a call is launched.  Dense calls with at least one full flash workgroup of (target, head) rows
// share source tiles between targets (flash kernel); every other call runs one workgroup per
// (target, 16 heads).  With a workspace, launches that would leave most of the 256 CUs idle split
// each target's sources into pieces (at least 4 tiles of 64 for the flash kernel, at least 4
// groups of 32 for the gather kernel) until the grid has about 512 (flash) or 256 (gather)
// workgroups.
struct SinkPlan {
  bool flash;
  int n_split;
  int nw;        // gather: waves per workgroup
  int64_t gps;   // gather: 32-source groups per piece
  size_t ws;     // bytes of piece results (0 without a split)
};

SinkPlan sink_plan(bool dense, int64_t B, int64_t T, int64_t H, int64_t S, int64_t K, bool may_split) {
  SinkPlan p{};
  p.n_split = 1;
  const int64_t rows = B * T;
  if (dense && T * H >= 64 && K > 0) {
    p.flash = true;
    const int64_t wgs = B * dense_flash_row_blocks(T, H);
    const int64_t tiles = ceil_div(S, dense_flash_tile());
    if (may_split && wgs < 512 && tiles >= 8)
      p.n_split = static_cast<int>(std::min<int64_t>(ceil_div(512, wgs), tiles / 4));
  } else {
    p.flash = false;
    const int64_t n_groups = ceil_div(K, kGroup);
    const int64_t wgs = rows * ceil_div(H, 16);
    if (may_split && wgs < 256 && n_groups > 4)
      p.n_split = static_cast<int>(std::min<int64_t>(ceil_div(256, wgs), ceil_div(n_groups, 4)));
    p.gps = std::max<int64_t>(ceil_div(n_groups, p.n_split), 1);
    if (p.n_split > 1) p.n_split = static_cast<int>(ceil_div(n_groups, p.gps));  // no empty pieces
    p.nw = p.gps >= 8 ? 8 : (p.gps >= 4 ? 4 : 2);
  }
  p.ws = p.n_split > 1 ? align_up(static_cast<size_t>(rows * H) * p.n_split * kPartStride * sizeof(float), 256) : 0;
  return p;
}

}  // namespace

bool sink_attention_mfma_supported(int32_t dtype, int64_t D) {
  return D == kD && (dtype == AEKV_BF16 || dtype == AEKV_F16);
}

size_t sink_attention_mfma_workspace(bool dense, int64_t B, int64_t T, int64_t H, int64_t S, int64_t K) {
  return sink_plan(dense, B, T, H, S, K, true).ws;
}

int sink_attention_mfma(const void* q, const void* kv, const void* idx, int idx_kind, const void* sink,
                        int sink_scalar, int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t S, int64_t K,
                        float scale, void* ws, size_t ws_bytes, void* out, hipStream_t st, const char* who) {
  const int64_t rows = B * T;
  const int64_t hgroups = ceil_div(H, 16);
  if (rows > 0x7fffffffLL || hgroups > 65535) return fail(AEKV_ERR_UNSUPPORTED, "%s: grid too large", who);
  if (rows == 0 || H == 0) return AEKV_OK;
  SinkPlan p = sink_plan(idx_kind == 0, B, T, H, S, K, ws != nullptr);
  if (p.ws > 0 && ws_bytes < p.ws)
    return fail(AEKV_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who, p.ws, ws_bytes);
  if (p.ws > 0 && !is_aligned(ws, 256)) return fail(AEKV_ERR_ALIGN, "%s: workspace must be 256-byte aligned", who);
  if (p.n_split > 65535) return fail(AEKV_ERR_UNSUPPORTED, "%s: too many source pieces", who);
  float* part = p.n_split > 1 ? static_cast<float*>(ws) : nullptr;
  if (p.flash) {
    if (int rc = launch_dense_flash_attention(q, kv, sink, sink_scalar, dtype, B, T, H, S, scale, p.n_split, part,
                                              out, st, who))
      return rc;
  } else {
    GatherArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.kv = static_cast<const uint16_t*>(kv);
    a.idx = idx;
    a.sink = static_cast<const uint16_t*>(sink);
    a.sink_scalar = sink_scalar;
    a.H = static_cast<int>(H);
    a.T = T;
    a.S = S;
    a.K = K;
    a.scale2 = scale * kLog2e;
    a.n_split = p.n_split;
    a.gps = p.gps;
    a.part = part;
    a.out = static_cast<uint16_t*>(out);
    const int hg = static_cast<int>(hgroups);
    if (dtype == AEKV_BF16) {
      if (idx_kind == 0) launch_gather_t<AEKV_BF16, 0>(a, rows, hg, p.nw, st);
      else if (idx_kind == 4) launch_gather_t<AEKV_BF16, 4>(a, rows, hg, p.nw, st);
      else launch_gather_t<AEKV_BF16, 8>(a, rows, hg, p.nw, st);
    } else {
      if (idx_kind == 0) launch_gather_t<AEKV_F16, 0>(a, rows, hg, p.nw, st);
      else if (idx_kind == 4) launch_gather_t<AEKV_F16, 4>(a, rows, hg, p.nw, st);
      else launch_gather_t<AEKV_F16, 8>(a, rows, hg, p.nw, st);
    }
    if (int rc = check_launch(who)) return rc;
  }
  if (p.n_split == 1) return AEKV_OK;
  const int64_t n = rows * H;
  const int nt = ceil_div(n, int64_t(8)) >= 256 ? 256 : 64;
  const int64_t n_wg = ceil_div(n, static_cast<int64_t>(nt / 32));
  if (n > 0x7fffffffLL) return fail(AEKV_ERR_UNSUPPORTED, "%s: too many rows", who);
  const dim3 grid(static_cast<uint32_t>(n_wg));
  const uint16_t* sk = static_cast<const uint16_t*>(sink);
  uint16_t* o = static_cast<uint16_t*>(out);
  const int hh = static_cast<int>(H);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(nt), 0, st, part, p.n_split, sk, sink_scalar, hh, static_cast<int>(n), o);
  };
  if (dtype == AEKV_BF16) {
    if (nt == 256) launch(sink_attn_combine_kernel<AEKV_BF16, 256>);
    else launch(sink_attn_combine_kernel<AEKV_BF16, 64>);
  } else {
    if (nt == 256) launch(sink_attn_combine_kernel<AEKV_F16, 256>);
    else launch(sink_attn_combine_kernel<AEKV_F16, 64>);
  }
  return check_launch(who);
}

}  // namespace aekv
