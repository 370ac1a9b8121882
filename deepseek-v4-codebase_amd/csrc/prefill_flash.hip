// Flash-style matrix-core sink attention in which the (target, head) query rows of a workgroup (64
// or 96) share every source tile, for two callers:
//   * chunked-prefill HCA attention over dequantised blocks (bf16, K = V: rows of 256 bytes);
//   * the dense drop-in tiled_prefill_attention (aether_kernels/sparse_attention.py:19-42, sink
//     counted once as in aether_2b/modeling.py:158-178) when a call has 64 or more (target, head)
//     rows: bf16 or fp16 kv [B, S, 2, 128], i.e. rows of 512 bytes holding K then V, every target
//     over every source.
// The description below is the HCA use; the dense one is the same kernel with no masks, one
// source buffer, tiles of 64 512-byte rows (the same 32 KB), V read from the second half of each
// row, and the fp16 products (v_mfma_f32_32x32x16_f16) for fp16 inputs.
//
// Reference: aether_2b/modeling.py:293-325 (_forward_tiled_prefill, HCA): target t attends blocks
// [0, g_t) and window entries [max(0, t - W + 1), t] with K = V and the per-head sink
// (sink_attention, modeling.py:158-178: the sink counted once in the normaliser).  The blocks are
// first decoded once per sequence to the bf16 values the engine attends (PolarQuant.decode,
// aekv_tq_decode), then this kernel runs over [blocks; window] with per-row masks:
//   row r = t * H + h of sequence b; source j < g_t (block) or window entry e in
//   [win_start_t, win_start_t + win_len_t).
//
// Work split.  A workgroup owns 32 RG consecutive rows (RG row groups of 32).  The sources of its
// targets (blocks [0, max g), window [min start, max end)) stream through LDS in tiles of TILE keys,
// row-major (key, 128 dims), in two alternating buffers (one barrier per tile), loaded by buffer
// loads that write LDS directly (no register staging), one tile ahead.  Wave w takes row group
// w % RG (32 rows, lane l holds row l % 32) and key split w / RG (TILE / KS keys) of every tile:
// with v_mfma_f32_32x32x16_bf16 every LDS byte feeds twice the matrix work of a 16-row wave.  The
// KS waves of a row group keep separate online-softmax states, merged once at the end through LDS.
// Shapes: RG = 2, KS = 2 (4 waves, two workgroups per CU) for both callers; RG = 3, KS = 4 (12
// waves, one workgroup and three waves per SIMD) for HCA when that balances the CUs better.
//
// Matrix layouts (v_mfma_f32_32x32x16_bf16, measured): A lane l holds A[l%32][8(l/32)+j], B lane l
// holds B[8(l/32)+j][l%32], D lane l register v holds D[8(v/4) + 4(l/32) + v%4][l%32].
//   S^T = K Q^T: m = key, n = row, k = dims 16 ks + 8 (l/32) + j.  A = 16-byte row chunks of the
//     tile, B = the row's query (registers).  Lane l gets the scores of keys
//     8q + 4(l/32) + r (q, r < 4) of each 32-key block for its row.
//   O^T += V^T P^T per 16-key chunk c: m = dim, n = row, k = key with lane half h = l/32 holding
//     keys {16c + 4h + j, 16c + 8 + 4h + j} (j < 4): exactly the lane's own scores, so P^T needs
//     no data movement.  A = V^T comes from the same row-major tile through the gfx950 transpose
//     load ds_read_b64_tr_b16 (lane i of a 16-lane group gets element i%4 of source lane
//     4j + i/4 as element j, measured): source lane s of the group points at key k_(s/4), dims
//     4(s%4)..+3 of the group's 16 dims, so every lane receives 4 keys of one dim.
//   Row chunks are stored XOR-swizzled, chunk c of key r at c ^ sigma(r % 16) with
//   sigma(r) = 4(r%4) + (r/4)%4: the 16 keys of a row-chunk read land on 16 distinct chunks, and
//   the 4 keys x 4 chunks of a 32-lane transpose pass on 16 distinct chunks (64 banks), no padding.
//
// Softmax in the exp2 domain with the exact running maximum, so a row's largest weight is exactly 1
// in bf16 and every weight ratio carries one bf16 rounding (a maximum raised only past a margin
// leaves two, which measurably exceeds the attention tolerance).  The rescale of O and l is a
// wave-uniform branch taken on tiles that raise some row's maximum.  The normaliser is the sum of
// the very bf16 weights the numerator used: each lane adds its own weights of the row with
// v_dot2_f32_bf16 (f16) against ones, and the two lane halves are added at the end.  Tiles that
// every row of the workgroup sees in full skip the masks.
#include <atomic>

#include "tq_device.h"

namespace aekv {
namespace {

constexpr int kFD = 128;
constexpr int kTileBytes = 32768;     // one LDS tile buffer
constexpr int kSlotFloats = 4096;     // one wave's merge state in LDS: O of 32 rows x 128 dims
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kFNegInf = -__builtin_inff();
constexpr int kBufWord3 = 0x00020000;  // buffer resource word 3: raw 32-bit data, range-checked

typedef __attribute__((ext_vector_type(8))) __bf16 fbf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 ff16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 fbf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 ff16x2_t;
typedef __attribute__((ext_vector_type(16))) float ff32x16_t;
typedef __attribute__((ext_vector_type(4))) short fi16x4_t;
typedef __attribute__((address_space(3))) fi16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

// Source rows of ROWB bytes: 256 (K = V) or 512 (K, then V).  A tile holds kTile rows (32 KB).
// A workgroup has RG groups of 32 query rows and splits every tile's keys KS ways: wave w takes
// row group w % RG and keys [kKW (w / RG), + kKW) of each tile.  Two shapes are instantiated:
// RG = 2, KS = 2 (4 waves, 64 rows, two workgroups per CU) and, for K = V rows, RG = 3, KS = 4
// (12 waves, 96 rows, one workgroup and three waves per SIMD).
template <int ROWB, int RG, int KS>
struct FlashGeom {
  static_assert(ROWB == 256 || ROWB == 512, "rows of K (= V) or of K then V");
  static_assert(KS == 2 || KS == 4, "the key splits merge pairwise");
  static_assert(RG * KS == 4 || RG * KS == 12, "4 waves (two workgroups per CU) or 12 (one)");
  static constexpr int kRowBytes = ROWB;
  static constexpr int kWaves = RG * KS, kThreads = 64 * kWaves, kRows = 32 * RG;
  static constexpr int kWavesPerSimd = kWaves == 4 ? 2 : 3;  // resident waves per SIMD (register budget)
  static constexpr int kTile = kTileBytes / ROWB;       // sources per tile (128 or 64)
  static constexpr int kKW = kTile / KS;                // sources per wave and tile
  static constexpr int kKB = kKW / 32;                  // 32-key score blocks per wave and tile
  static constexpr int kLoadWaves = kWaves < 8 ? kWaves : 8;  // waves that stage the tiles
  static constexpr int kPass = 1024 * kLoadWaves;       // bytes of a tile per staging pass
  static constexpr int kChunks = kTileBytes / kPass;    // staging passes per tile
  static constexpr int kVOff = ROWB == 256 ? 0 : 256;   // V's byte offset in a row
  static constexpr bool kSplit = ROWB == 512;           // the dense caller may split a row's sources
  static constexpr int kSlots = RG * KS / 2;            // merge states in LDS at once (16 KB each)
  static constexpr int kMergeExtra = kSlots > 4 ? (kSlots - 4) * kSlotFloats * 4 : 16;  // beyond the tiles
  static_assert(kKB >= 1 && kKW % 32 == 0, "tiles are whole 32-key blocks per wave");
  static_assert(kTileBytes % kPass == 0 && kPass % ROWB == 0, "whole rows per staging pass");
  static_assert(kSlots <= 6, "merge slots");
};

// The element type's matrix instruction, weight rounding and constants.
template <int DT>
struct FlashElem;
template <>
struct FlashElem<AEKV_BF16> {
  typedef fbf16x8_t v8;
  static constexpr uint32_t kOnePair = 0x3F803F80u;
  __device__ static ff32x16_t mma(v8 a, v8 b, ff32x16_t c) { return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0); }
  __device__ static uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
  // c + the two values of a packed pair (products with 1.0 are exact)
  __device__ static float add_pair(uint32_t pr, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(fbf16x2_t, pr), __builtin_bit_cast(fbf16x2_t, kOnePair), c,
                                           false);
  }
};
template <>
struct FlashElem<AEKV_F16> {
  typedef ff16x8_t v8;
  static constexpr uint32_t kOnePair = 0x3C003C00u;
  __device__ static ff32x16_t mma(v8 a, v8 b, ff32x16_t c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }
  __device__ static uint32_t pack(float lo, float hi) { return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16); }
  __device__ static float add_pair(uint32_t pr, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(ff16x2_t, pr), __builtin_bit_cast(ff16x2_t, kOnePair), c, false);
  }
};

// chunk c of key r sits at c ^ chunk_swizzle(r % 16) of its 256-byte LDS row
__device__ __forceinline__ int chunk_swizzle(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

template <int N>
struct IntC {
  static constexpr int value = N;
};

template <int HL>
__device__ __forceinline__ int xor_lane_i(int v) {
  return __builtin_bit_cast(int, xor_lane<HL>(__builtin_bit_cast(float, v)));
}
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, xor_lane_i<1>(v));
  v = max(v, xor_lane_i<2>(v));
  v = max(v, xor_lane_i<4>(v));
  v = max(v, xor_lane_i<8>(v));
  v = max(v, xor_lane_i<16>(v));
  return max(v, xor_lane_i<32>(v));
}
__device__ __forceinline__ int wave_min_i(int v) {
  v = min(v, xor_lane_i<1>(v));
  v = min(v, xor_lane_i<2>(v));
  v = min(v, xor_lane_i<4>(v));
  v = min(v, xor_lane_i<8>(v));
  v = min(v, xor_lane_i<16>(v));
  return min(v, xor_lane_i<32>(v));
}

__device__ __forceinline__ fi16x4_t lds_read_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
}

struct FlashArgs {
  const uint16_t* q;      // [B, T, H, 128]
  const uint16_t* kblk;   // [B, S, ROWB / 2]: dequantised blocks (K = V), or kv [B, S, 2, 128]
  const uint16_t* win;    // [B, Wt, ROWB / 2] or null (Wt = 0)
  const int32_t* vis;     // [B * T] or null (all S)
  const int32_t* wstart;  // [B * T] or null (0)
  const int32_t* wlen;    // [B * T] or null (to the end of the window)
  const void* sink;       // [H] or [1] of sink_dt (f32, or the input type)
  int sink_dt, sink_scalar;
  int64_t S, Wt;
  int T;
  uint32_t gx;            // workgroups per sequence
  int H;
  float scale2;           // softmax scale * log2(e)
  int n_split;            // source pieces per row block (1: the workgroup finishes its rows)
  float* part;            // [B * T * H, n_split, 132]: max, sum (log2 units), 2 pad, O[128]
  uint16_t* out;          // [B, T, H, 128]
};

// Two waves per SIMD (at most 256 registers per lane): the accumulators stay in VGPRs across the
// loop (the matrix instructions take VGPR operands) instead of moving to AGPRs and back, and the
// scheduler may spend registers on reading LDS operands ahead of the products.  A launch has about
// 1.5 workgroups per CU at the bench shape, so more resident waves would not exist anyway.
template <int DT, int ROWB, int RG, int KS>
__global__ __launch_bounds__(64 * RG * KS) __attribute__((
    amdgpu_waves_per_eu(FlashGeom<ROWB, RG, KS>::kWavesPerSimd, FlashGeom<ROWB, RG, KS>::kWavesPerSimd))) void
flash_sink_attn_kernel(FlashArgs a) {
  using Gm = FlashGeom<ROWB, RG, KS>;
  using E = FlashElem<DT>;
  using v8 = typename E::v8;
  constexpr int kRowBytes = Gm::kRowBytes, kFTile = Gm::kTile, kKW = Gm::kKW, kKB = Gm::kKB;
  constexpr int kChunks = Gm::kChunks, kVOff = Gm::kVOff, kPass = Gm::kPass, kWaves = Gm::kWaves;
  // the two tile buffers, [key][swizzled 16-byte chunks]: separate arrays, so that the compiler
  // sees that the loads into one do not write what is read from the other
  __shared__ __align__(16) uint8_t Ls0[kTileBytes];
  __shared__ __align__(16) uint8_t Ls1[kTileBytes];
  __shared__ __align__(16) uint8_t Lm[Gm::kMergeExtra];  // merge slots beyond the tile buffers
  __shared__ int s_rng[kWaves][4];                     // per wave: max blocks, min blocks, window lo, hi
  __shared__ float s_ml[Gm::kSlots][2][64];            // (m, l) of the merge slots per lane

  // Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2): renumber them so
  // that XCD x runs the consecutive range [x n/8, (x+1) n/8), i.e. whole sequences, whose blocks
  // then stay in that XCD's L2 instead of every L2 streaming every sequence.
  // (32-bit index arithmetic: the launcher bounds the grid and B * T * H below 2^31)
  const uint32_t n_wg = gridDim.x;
  uint32_t wgi = blockIdx.x;
  if (n_wg % 8 == 0) wgi = (wgi % 8) * (n_wg / 8) + wgi / 8;
  const uint32_t nsp = Gm::kSplit ? static_cast<uint32_t>(a.n_split) : 1u;
  const uint32_t per_seq = a.gx * nsp;
  const int b = static_cast<int>(wgi / per_seq);
  const int wrow = static_cast<int>((wgi % per_seq) / nsp);
  const int split = static_cast<int>(wgi % nsp);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (a scalar register)
  const int rh = wv % RG, kh = wv / RG;  // row group, key split
  const int rl = lane & 31, hh = lane >> 5;
  const int H = a.H;
  const int RT = a.T * H;
  const int r = wrow * Gm::kRows + 32 * rh + rl;  // this lane's row
  const bool rv = r < RT;
  const int t = rv ? static_cast<int>(static_cast<uint32_t>(r) / static_cast<uint32_t>(H)) : 0;
  const int h = rv ? r - t * H : 0;
  const int64_t bt = static_cast<int64_t>(b) * a.T + t;

  // Every load of the prologue is issued before any is used (one memory round): the row's source
  // counts first, then its query (lanes past the rows read row 0 and use zeros), so that the
  // bounds' wait leaves the query loads in flight.
  // (absent counts: all S blocks, window from 0 to its end)
  const int32_t c_vis = load_or(a.vis, bt, a.q, 0x7fffffff), c_ws = load_or(a.wstart, bt, a.q, 0);
  const int32_t c_wl = load_or(a.wlen, bt, a.q, 0x7fffffff);
  uint4 qv[8];
  {
    const uint16_t* qp = a.q + (static_cast<int64_t>(b) * RT + (rv ? r : 0)) * kFD + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qv[ks] = *reinterpret_cast<const uint4*>(qp + 16 * ks);
  }
  // the row's sources: blocks [0, nb), window entries [w0, w1) (computed for every lane, then
  // masked: a branch on rv would take the count loads, and their wait, into it)
  const int nb_r = static_cast<int>(min<int64_t>(max(c_vis, 0), a.S));
  const int w0_r = static_cast<int>(min<int64_t>(max(c_ws, 0), a.Wt));
  const int wl_r = static_cast<int>(min<int64_t>(max(c_wl, 0), a.Wt - w0_r));
  const int nb = rv ? nb_r : 0, w0 = rv ? w0_r : 0, w1 = rv ? w0_r + wl_r : 0;
  // the workgroup's bounds: reduced within each wave, then over the 4 waves through LDS
  {
    const bool hw = rv && w1 > w0;
    const int v0 = wave_max_i(rv ? nb : 0), v1 = wave_min_i(rv ? nb : 0x7fffffff);
    const int v2 = wave_min_i(hw ? w0 : 0x7fffffff), v3 = wave_max_i(hw ? w1 : 0);
    if (lane == 0) {
      s_rng[wv][0] = v0;
      s_rng[wv][1] = v1;
      s_rng[wv][2] = v2;
      s_rng[wv][3] = v3;
    }
  }
  __syncthreads();
  int gmax = 0, nbmin = 0x7fffffff, wlo = 0x7fffffff, whi = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    gmax = max(gmax, s_rng[w][0]);
    nbmin = min(nbmin, s_rng[w][1]);
    wlo = min(wlo, s_rng[w][2]);
    whi = max(whi, s_rng[w][3]);
  }
  // workgroup-uniform (readfirstlane keeps them in scalar registers)
  gmax = __builtin_amdgcn_readfirstlane(gmax);
  nbmin = __builtin_amdgcn_readfirstlane(nbmin);
  whi = __builtin_amdgcn_readfirstlane(whi);
  wlo = whi > 0 ? __builtin_amdgcn_readfirstlane(wlo) : 0;
  const int n_bt = (gmax + kFTile - 1) / kFTile;
  const int n_wt = whi > wlo ? (whi - wlo + kFTile - 1) / kFTile : 0;
  const int n_tiles = n_bt + n_wt;
  // this workgroup's tiles [it0, it1): one piece of n_split
  const int tps = (n_tiles + static_cast<int>(nsp) - 1) / static_cast<int>(nsp);
  const int it0 = min(split * tps, n_tiles), it1 = min(it0 + tps, n_tiles);

  // the row's query as the B operand of S^T = K Q^T: dims 16 ks + 8 hh .. + 7
  v8 qb[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) qb[ks] = __builtin_bit_cast(v8, rv ? qv[ks] : make_uint4(0u, 0u, 0u, 0u));
  // the queries have landed before any tile load is issued: otherwise the wait for them, merged
  // over the loop's back edge, becomes a wait for every tile load on every iteration
  __builtin_amdgcn_s_waitcnt(0);

  // LDS byte offsets per lane (the tile and block offsets are multiples of 16 keys, which leave
  // the swizzle unchanged, and become immediates).  The swizzle permutes the 16 chunks of each
  // 256-byte half of a row.
  //   Row-chunk reads (K): key kKW kh + 32 kb + rl, chunk (2 ks + hh) ^ sigma(rl % 16), i.e.
  //   byte sA ^ 32 ks with sA = row | 32 (sigma >> 1) | 16 (hh ^ sigma & 1) (the row's byte offset
  //   is a multiple of 256, so the chunk bits are free).
  //   Transpose reads (V, 16-lane group G = lane / 16, s = lane % 16): key kKW kh + 16 c + 4 hh +
  //   s / 4 + 8 e, dims 32 mb + 16 (G % 2) + 4 (s % 4) .. + 3, i.e. chunk 4 mb + x with
  //   x = 2 (G % 2) + (s % 4) / 2, xor sigma(key) = 4 (s / 4) + (hh | 2 e): byte
  //   (tA ^ 64 mb ^ 32 e) + 8 e ROWB with tA = row(e = 0) + V offset | 64 (s / 4) | 16 (x ^ hh) | 8 (s % 2).
  // Two registers instead of 16 offsets; the xors are recomputed per tile where registers are short.
  const int kbase = kKW * kh * kRowBytes;
  int sA, tA;
  {
    const int sg = chunk_swizzle(rl & 15);
    sA = (kbase + rl * kRowBytes) | ((sg >> 1) << 5) | ((hh ^ (sg & 1)) << 4);
    const int s16 = lane & 15, G = lane >> 4;
    const int x = 2 * (G & 1) + ((s16 & 3) >> 1);
    tA = (kbase + (4 * hh + (s16 >> 2)) * kRowBytes + kVOff) | ((s16 >> 2) << 6) | ((x ^ hh) << 4) | ((s16 & 1) << 3);
  }

  const uint8_t* kseq = reinterpret_cast<const uint8_t*>(a.kblk) + static_cast<int64_t>(b) * a.S * kRowBytes;
  const uint8_t* wseq = reinterpret_cast<const uint8_t*>(a.win) + static_cast<int64_t>(b) * a.Wt * kRowBytes;
  // Staging straight into LDS (buffer loads with the LDS bit) by the first kLoadWaves waves
  // (P = 1024 kLoadWaves bytes per pass): pass c of wave wv writes bytes [P c + 1024 wv, + 1024) of
  // the tile buffer, lane l at + 16 l, so lane l loads the global chunk that the swizzle puts there:
  // key k = (P c + 1024 wv + 16 l) / ROWB, slot j = (1024 wv + 16 l) % ROWB / 16 of it, i.e. chunk
  // (j & 16) + ((j & 15) ^ sigma(k % 16)).  The pass's keys start at a multiple of P / ROWB keys
  // (8, 16 or 32), so the offsets repeat with period 2 or 1 in c; P c goes in the scalar offset.
  int voff[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int lin = 1024 * wv + 16 * lane;
    const int kin = lin / kRowBytes, slot = (lin % kRowBytes) / 16;
    const int ksw = ((kPass / kRowBytes) * p + kin) & 15;
    voff[p] = kin * kRowBytes + 16 * ((slot & 16) + ((slot & 15) ^ chunk_swizzle(ksw)));
  }
  // tile it into LDS buffer buf: keys [base, base + TILE) of the blocks (it < n_bt) or of the
  // window, read through a buffer resource whose range ends at the workgroup's last source, so that
  // the rows past it are zero (never attended) without a branch or an access.  A tile past the last
  // has an empty range: its loads are issued (no branch, so the wait counts stay exact) but touch
  // no memory.
  // (the tile bounds are captured by value: selecting between two captured references puts them
  // in scratch memory)
  auto load_tile = [&, gmax, whi, wlo, n_bt, it1, kseq, wseq](int it, auto buf_c) {
    uint8_t* const dst = decltype(buf_c)::value ? Ls1 : Ls0;
    const bool blk = it < n_bt;
    const int base = blk ? it * kFTile : wlo + (it - n_bt) * kFTile;
    const int lim = blk ? gmax : whi;
    const uint8_t* src = (blk ? kseq : wseq) + static_cast<int64_t>(it < it1 ? base : 0) * kRowBytes;
    const int n_bytes = it < it1 ? min(lim - base, kFTile) * kRowBytes : 0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), 0, n_bytes, kBufWord3);
    if (Gm::kLoadWaves == kWaves || wv < Gm::kLoadWaves) {
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(dst + kPass * c + 1024 * wv), 16, voff[c & 1],
                                                 kPass * c, 0, 0);
    }
  };

  // m_run: the row's running maximum over this wave's keys, in scaled log2 units (the same in both
  // lane halves).  lsum: the sum of this lane's bf16 weights of the row (its half of the keys).
  float m_run = kFNegInf, lsum = 0.0f;
  ff32x16_t O[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) O[mb] = ff32x16_t{};

  // Each tile is loaded into the other LDS buffer while the current one is used; its loads have
  // landed (this wave's: the wait; every wave's: the barrier) before the step that reads it.  The
  // compiler does not track the LDS writes of these loads, so both waits are explicit.
  load_tile(it0, IntC<0>{});
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // one tile; the buffer index is a compile-time constant (LDS offsets are immediates)
  auto step = [&](int it, auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;  // LDS buffer of tile it
    load_tile(it + 1, IntC<buf ^ 1>{});  // the other buffer was last read before the previous barrier
    const uint8_t* lt = buf ? Ls1 : Ls0;
    int sa = sA, ta = tA;
    if constexpr (Gm::kWavesPerSimd > 2) asm volatile("" : "+v"(sa), "+v"(ta));  // not hoisted: recomputed per tile

    // S^T for keys 32 kb + 8 q + 4 hh + r of this wave's half tile, row rl (s[kb][4 q + r])
    ff32x16_t s[kKB];
    {
      uint4 kv[kKB][8];  // every row chunk of the half tile read before the products
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) kv[kb][ks] = *reinterpret_cast<const uint4*>(lt + 32 * kRowBytes * kb + (sa ^ (ks << 5)));
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb) {
        s[kb] = ff32x16_t{};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) s[kb] = E::mma(__builtin_bit_cast(v8, kv[kb][ks]), qb[ks], s[kb]);
      }
    }
    // masks (only where some row of the workgroup does not see the whole tile)
    const bool blk_tile = it < n_bt;
    const int base = blk_tile ? it * kFTile : wlo + (it - n_bt) * kFTile;
    float tmax = kFNegInf;
    if (blk_tile && base + kFTile <= nbmin) {
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) tmax = fmaxf(tmax, s[kb][v]);
    } else {
      // this row's keys of the wave's half tile: [lo, hi) relative to its first key
      const int k0 = base + kKW * kh;
      const int lo = (blk_tile ? 0 : w0) - k0, hi = (blk_tile ? nb : w1) - k0;
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int k = 32 * kb + 8 * (v >> 2) + 4 * hh + (v & 3);
          s[kb][v] = (k >= lo && k < hi) ? s[kb][v] : kFNegInf;
          tmax = fmaxf(tmax, s[kb][v]);
        }
    }
    tmax = fmaxf(tmax, xor_lane<32>(tmax));
    const float mt = tmax * a.scale2;
    if (__builtin_amdgcn_ballot_w64(mt > m_run)) {  // some row's maximum moved up
      const float m_new = fmaxf(m_run, mt);
      const float alpha = m_new == kFNegInf ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      lsum *= alpha;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) O[mb] *= alpha;
      m_run = m_new;
    }
    const float nm = m_run == kFNegInf ? 0.0f : -m_run;
    // O^T[dims 32 mb + ..][row rl] += V^T P^T per 16-key chunk c of each block
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = __builtin_amdgcn_exp2f(fmaf(s[kb][8 * c + j], a.scale2, nm));
        const uint4 pw = make_uint4(E::pack(p[0], p[1]), E::pack(p[2], p[3]), E::pack(p[4], p[5]), E::pack(p[6], p[7]));
        const v8 pb = __builtin_bit_cast(v8, pw);
        lsum = E::add_pair(pw.w, E::add_pair(pw.z, E::add_pair(pw.y, E::add_pair(pw.x, lsum))));
        v8 va[4];  // the chunk's V^T operands, read before their products
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          const uint8_t* q0 = lt + (32 * kb + 16 * c) * kRowBytes;
          const fi16x4_t lo4 = lds_read_tr16(q0 + (ta ^ (mb << 6)));
          const fi16x4_t hi4 = lds_read_tr16(q0 + 8 * kRowBytes + (ta ^ (mb << 6) ^ 32));
          va[mb] = __builtin_bit_cast(v8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
        }
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) O[mb] = E::mma(va[mb], pb, O[mb]);
      }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };
  // unrolled over the two buffers so that both indices are constants (a skipped second step
  // leaves the loop, so it does not blur the wait counts on the back edge)
#pragma unroll 1
  for (int it = it0; it < it1; it += 2) {
    step(it, IntC<0>{});
    if (it + 1 < it1) step(it + 1, IntC<1>{});
  }
  lsum += xor_lane<32>(lsum);  // the row's sum over both lane halves

  // Merge the KS key splits of each row group through LDS (the tile buffers, free after the last
  // barrier, then Lm), pairwise: split 2j + 1 writes its (m, l, O) to a slot and split 2j folds it
  // in; with four splits, split 2 then hands its result to split 0.  Split 0 writes the rows.
  auto slot = [&](int i) -> float* {  // [mb][v][lane]
    return i < 2 ? reinterpret_cast<float*>(Ls0) + kSlotFloats * i
           : i < 4 ? reinterpret_cast<float*>(Ls1) + kSlotFloats * (i - 2)
                   : reinterpret_cast<float*>(Lm) + kSlotFloats * (i - 4);
  };
  auto put = [&](int i) {
    float* ob = slot(i);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) ob[(mb * 16 + v) * 64 + lane] = O[mb][v];
    s_ml[i][0][lane] = m_run;
    s_ml[i][1][lane] = lsum;
  };
  auto fold = [&](int i) {
    const float* ob = slot(i);
    const float m1 = s_ml[i][0][lane], l1 = s_ml[i][1][lane];
    const float mm = fmaxf(m_run, m1);
    const float f0 = m_run == kFNegInf ? 0.0f : exp2f(m_run - mm);
    const float f1 = m1 == kFNegInf ? 0.0f : exp2f(m1 - mm);
    lsum = lsum * f0 + l1 * f1;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) O[mb][v] = O[mb][v] * f0 + ob[(mb * 16 + v) * 64 + lane] * f1;
    m_run = mm;
  };
  {
    const int pslot = rh * (KS / 2) + (kh >> 1);
    if (kh & 1) put(pslot);
    __syncthreads();
    if (!(kh & 1)) fold(pslot);
    if constexpr (KS == 4) {
      __syncthreads();  // every fold above has read its slot
      if (kh == 2) put(rh * 2);
      __syncthreads();
      if (kh == 0) fold(rh * 2);
    }
  }
  if (kh != 0 || !rv) return;
  if (Gm::kSplit && nsp > 1) {
    // one piece: the row's (max, sum, O) relative to its max, merged with the sink by the combine
    float* dst = a.part + ((static_cast<int64_t>(b) * RT + r) * a.n_split + split) * (kFD + 4);
    if (hh == 0) {
      dst[0] = m_run;
      dst[1] = lsum;
    }
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4*>(dst + 4 + 32 * mb + 8 * q + 4 * hh) =
            make_float4(O[mb][4 * q], O[mb][4 * q + 1], O[mb][4 * q + 2], O[mb][4 * q + 3]);
    return;
  }
  // the sink, counted once: out = O / (l + e^{sink - m}) with m = max(m_run, sink)
  const int sh = a.sink_scalar ? 0 : h;
  const float skv = a.sink_dt == AEKV_F32   ? static_cast<const float*>(a.sink)[sh]
                    : a.sink_dt == AEKV_F16 ? f16_to_f32(static_cast<const uint16_t*>(a.sink)[sh])
                                            : bf16_to_f32(static_cast<const uint16_t*>(a.sink)[sh]);
  const float sk = skv * kLog2e;
  const float mf = fmaxf(m_run, sk);
  const float fo = m_run == kFNegInf ? 0.0f : exp2f(m_run - mf);
  const float L = fmaf(lsum, fo, exp2f(sk - mf));
  const float rs = mf == kFNegInf ? 0.0f : fo / L;  // no source and sink -inf: 0
  uint16_t* orow = a.out + (static_cast<int64_t>(b) * RT + r) * kFD;  // r < RT here
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = O[mb][4 * q + i] * rs;
      *reinterpret_cast<uint2*>(orow + 32 * mb + 8 * q + 4 * hh) = make_uint2(E::pack(o[0], o[1]), E::pack(o[2], o[3]));
    }
}

}  // namespace

size_t hca_prefill_flash_workspace(int64_t B, int64_t S) {
  return align_up(static_cast<size_t>(B) * static_cast<size_t>(S) * kFD * 2, 256);
}

bool hca_prefill_flash_supported(int64_t H, int64_t D) { return D == kFD && H >= 1; }

namespace {

using HcaNarrow = FlashGeom<256, 2, 2>;  // 64 rows, 4 waves
using HcaWide = FlashGeom<256, 3, 4>;    // 96 rows, 12 waves
using DenseGeom = FlashGeom<512, 2, 2>;

// Grid and index limits shared by both callers; fills the launch fields of a.
int flash_prepare(FlashArgs& a, int64_t B, int64_t T, int64_t H, int64_t S, int64_t Wt, int tile, int rows,
                  float softmax_scale, const char* who) {
  const int64_t RT = T * H;
  const int64_t gx = ceil_div(RT, rows);
  if (gx * B > 0x7fffffff || RT > 0x7fffffff - rows) return fail(AEKV_ERR_UNSUPPORTED, "%s: grid too large", who);
  if (S > 0x7fffffff - tile || Wt > 0x7fffffff - tile)
    return fail(AEKV_ERR_UNSUPPORTED, "%s: %lld sources / %lld window entries exceed the int32 indexing", who,
                (long long)S, (long long)Wt);
  a.T = static_cast<int>(T);
  a.S = S;
  a.Wt = Wt;
  a.H = static_cast<int>(H);
  a.scale2 = softmax_scale * kLog2e;
  a.gx = static_cast<uint32_t>(gx);
  return AEKV_OK;
}

std::atomic<int> g_hca_rows{0};  // 0: chosen per launch; 64 or 96: forced (aekv_set_flash_rows)

// Compute units of the current device (cached per device).
int64_t device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64) {
    if (const int c = cached[dev].load(std::memory_order_relaxed)) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev < 64) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace

// The 96-row shape when it leaves fewer rows on the busiest CU: two 64-row workgroups or one
// 96-row workgroup per CU at a time (e.g. 8 x 3072 rows: 384 narrow workgroups put 128 rows on
// half of the 256 CUs; 256 wide ones put 96 on each).
bool hca_flash_wide(int64_t B, int64_t T, int64_t H) {
  const int forced = g_hca_rows.load(std::memory_order_relaxed);
  if (forced) return forced == HcaWide::kRows;
  const int64_t cus = device_cus();
  const int64_t n_narrow = B * ceil_div(T * H, HcaNarrow::kRows), n_wide = B * ceil_div(T * H, HcaWide::kRows);
  return ceil_div(n_wide, cus) * HcaWide::kRows < ceil_div(n_narrow, 2 * cus) * 2 * HcaNarrow::kRows;
}

int launch_hca_prefill_flash(const void* q, const void* kblk, const void* window, const int32_t* vis,
                             const int32_t* wstart, const int32_t* wlen, const float* sink, int64_t B, int64_t T,
                             int64_t H, int64_t S, int64_t Wt, float softmax_scale, void* out, hipStream_t st,
                             const char* who) {
  FlashArgs a{};
  const bool wide = hca_flash_wide(B, T, H);
  const int rows = wide ? HcaWide::kRows : HcaNarrow::kRows;
  if (int rc = flash_prepare(a, B, T, H, S, Wt, HcaNarrow::kTile, rows, softmax_scale, who)) return rc;
  if (T * H == 0 || B == 0) return AEKV_OK;
  a.q = static_cast<const uint16_t*>(q);
  a.kblk = static_cast<const uint16_t*>(kblk);
  a.win = static_cast<const uint16_t*>(window);
  a.vis = vis;
  a.wstart = wstart;
  a.wlen = wlen;
  a.sink = sink;
  a.sink_dt = AEKV_F32;
  a.sink_scalar = 0;
  a.n_split = 1;
  a.out = static_cast<uint16_t*>(out);
  const dim3 grid(a.gx * static_cast<uint32_t>(B));
  if (wide) hipLaunchKernelGGL((flash_sink_attn_kernel<AEKV_BF16, 256, 3, 4>), grid, dim3(HcaWide::kThreads), 0, st, a);
  else hipLaunchKernelGGL((flash_sink_attn_kernel<AEKV_BF16, 256, 2, 2>), grid, dim3(HcaNarrow::kThreads), 0, st, a);
  return check_launch(who);
}

int64_t dense_flash_row_blocks(int64_t T, int64_t H) { return ceil_div(T * H, DenseGeom::kRows); }
int64_t dense_flash_tile() { return DenseGeom::kTile; }

int launch_dense_flash_attention(const void* q, const void* kv, const void* sink, int sink_scalar, int32_t dtype,
                                 int64_t B, int64_t T, int64_t H, int64_t S, float softmax_scale, int n_split,
                                 float* part, void* out, hipStream_t st, const char* who) {
  FlashArgs a{};
  if (int rc = flash_prepare(a, B, T, H, S, 0, DenseGeom::kTile, DenseGeom::kRows, softmax_scale, who)) return rc;
  if (T * H == 0 || B == 0) return AEKV_OK;
  if (n_split < 1 || (n_split > 1 && !part)) return fail(AEKV_ERR_VALUE, "%s: bad source split", who);
  if (static_cast<int64_t>(a.gx) * B * n_split > 0x7fffffff) return fail(AEKV_ERR_UNSUPPORTED, "%s: grid too large", who);
  a.n_split = n_split;
  a.part = part;
  a.q = static_cast<const uint16_t*>(q);
  a.kblk = static_cast<const uint16_t*>(kv);
  a.sink = sink;
  a.sink_dt = dtype;
  a.sink_scalar = sink_scalar;
  a.out = static_cast<uint16_t*>(out);
  const dim3 grid(a.gx * static_cast<uint32_t>(B) * static_cast<uint32_t>(n_split));
  if (dtype == AEKV_F16)
    hipLaunchKernelGGL((flash_sink_attn_kernel<AEKV_F16, 512, 2, 2>), grid, dim3(DenseGeom::kThreads), 0, st, a);
  else hipLaunchKernelGGL((flash_sink_attn_kernel<AEKV_BF16, 512, 2, 2>), grid, dim3(DenseGeom::kThreads), 0, st, a);
  return check_launch(who);
}

}  // namespace aekv

extern "C" int aekv_set_flash_rows(int rows) {
  if (rows != 0 && rows != aekv::HcaNarrow::kRows && rows != aekv::HcaWide::kRows)
    return aekv::fail(AEKV_ERR_VALUE, "aekv_set_flash_rows: rows must be 0, 64 or 96, got %d", rows);
  return aekv::g_hca_rows.exchange(rows);
}
