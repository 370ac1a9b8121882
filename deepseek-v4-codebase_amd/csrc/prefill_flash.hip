// Chunked-prefill HCA attention over dequantised blocks: a flash-style bf16 matrix-core kernel in
// which 64 (target, head) query rows share every source tile.
//
// Reference: aether_2b/modeling.py:293-325 (_forward_tiled_prefill, HCA): target t attends blocks
// [0, g_t) and window entries [max(0, t - W + 1), t] with K = V and the per-head sink
// (sink_attention, modeling.py:158-178: the sink counted once in the normaliser).  The blocks are
// first decoded once per sequence to the bf16 values the engine attends (PolarQuant.decode,
// aekv_tq_decode), then this kernel runs over [blocks; window] with per-row masks:
//   row r = t * H + h of sequence b; source j < g_t (block) or window entry e in
//   [win_start_t, win_start_t + win_len_t).
//
// A workgroup (4 waves) owns 64 consecutive rows, each wave 16 (one per lane column c16).  The
// sources of the workgroup's targets (blocks [0, max g), window [min start, max end)) stream
// through LDS in tiles of TILE keys, row-major (key, 128 dims), in two alternating buffers: the
// next tile is loaded into registers while the current one is multiplied, one barrier per tile.
// The same tile is both operands: S^T = K Q^T reads 16-byte row chunks (v_mfma_f32_16x16x32_bf16,
// keys x rows), and O^T += V^T P^T reads V^T with the gfx950 transpose load ds_read_b64_tr_b16,
// which hands lane i of each 16-lane group element j of source lane 4j + i/4's 4 halfwords
// (element i%4): source lane s of group g points at key 4g + s/4, dims 4(s%4)..+3 of a 16-dim
// block, so every lane receives 4 keys of one dim.  Row chunks are XOR-swizzled by key
// (chunk_swizzle) so that both the 16-lane row-chunk reads (16 keys, one chunk) and the transpose
// reads (8 keys x 32 bytes per 32-lane pass) hit distinct banks, with no padding.
//
// Softmax in the exp2 domain with the exact running maximum (so a row's largest weight is exactly
// 1 in bf16, as in a two-pass softmax); the rescale of O and l is a wave-uniform branch taken only
// on tiles that raise some row's maximum, which after the first few tiles is rare.  Tiles that
// every row of the workgroup sees in full skip the masks.
#include "tq_device.h"

namespace aekv {
namespace {

constexpr int kFD = 128;
constexpr int kFThreads = 256;        // 4 waves
constexpr int kFRows = 64;            // query rows per workgroup (16 per wave)
constexpr int kRowBytes = kFD * 2;    // one key of the tile in LDS
#ifndef AEKV_FLASH_TILE
#define AEKV_FLASH_TILE 64
#endif
#ifndef AEKV_FLASH_SWZ
#define AEKV_FLASH_SWZ 64
#endif
constexpr int kFTile = AEKV_FLASH_TILE;  // sources per tile
constexpr int kChunks = kFTile / 16;     // 16-byte chunks per thread and tile
constexpr int kTileBytes = kFTile * kRowBytes;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kFNegInf = -__builtin_inff();
static_assert(kFTile % 32 == 0 && kFTile <= 128, "tiles are whole 32-key chunks");
constexpr int kBufWord3 = 0x00020000;  // buffer resource word 3: raw 32-bit data, range-checked

typedef __attribute__((ext_vector_type(8))) __bf16 fbf16x8_t;
typedef __attribute__((ext_vector_type(4))) float ff32x4_t;
typedef __attribute__((ext_vector_type(4))) short fi16x4_t;
typedef __attribute__((address_space(3))) fi16x4_t lds_i16x4_t;

// Position of 16-byte chunk c of key r in its 256-byte LDS row: c ^ chunk_swizzle(r % 16).  A
// bijection on the 16 keys of a row-chunk read, and for the 8 keys of a transpose-read pass it
// sends chunk pairs {2n, 2n+1} to 8 distinct pairs (64 banks of 4 bytes).  AEKV_FLASH_SWZ=32
// selects the layout that is conflict-free for 32 banks instead.
__device__ __forceinline__ int chunk_swizzle(int r) {
#if AEKV_FLASH_SWZ == 32
  return ((r & 3) << 1) | ((r >> 2) & 1) | (r & 8);
#else
  return ((r & 7) << 1) | (r >> 3);
#endif
}

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
  const uint16_t* q;      // [B, T, H, 128] bf16
  const uint16_t* kblk;   // [B, S, 128] bf16 (dequantised blocks)
  const uint16_t* win;    // [B, Wt, 128] bf16
  const int32_t* vis;     // [B * T] or null (all S)
  const int32_t* wstart;  // [B * T] or null (0)
  const int32_t* wlen;    // [B * T] or null (to the end of the window)
  const float* sink;      // [H]
  int64_t S, Wt;
  int T;
  uint32_t gx;            // workgroups per sequence
  int H;
  float scale2;           // softmax scale * log2(e)
  uint16_t* out;          // [B, T, H, 128] bf16
};

// Two waves per SIMD (at most 256 registers per lane): the accumulators then stay in VGPRs across
// the loop (the matrix instructions take VGPR operands) instead of moving to AGPRs and back, and
// the scheduler may spend registers on reading LDS operands ahead of the products.  A launch has
// about 1.5 workgroups per CU at the bench shape, so more resident waves would not exist anyway.
__global__ __launch_bounds__(kFThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void hca_prefill_flash_kernel(
    FlashArgs a) {
  __shared__ __align__(16) uint8_t Ls[2][kTileBytes];  // [buffer][key][swizzled 16-byte chunks]
  __shared__ int s_rng[4][4];  // per wave: max blocks, min blocks, window lo, window hi

  // Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2): renumber them so
  // that XCD x runs the consecutive range [x n/8, (x+1) n/8), i.e. whole sequences, whose blocks
  // then stay in that XCD's L2 instead of every L2 streaming every sequence.
  // (32-bit index arithmetic: the launcher bounds the grid and B * T * H below 2^31)
  const uint32_t n_wg = gridDim.x;
  uint32_t wgi = blockIdx.x;
  if (n_wg % 8 == 0) wgi = (wgi % 8) * (n_wg / 8) + wgi / 8;
  const int b = static_cast<int>(wgi / a.gx);
  const int wrow = static_cast<int>(wgi % a.gx);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, c16 = lane & 15;
  const int H = a.H;
  const int RT = a.T * H;
  const int r = wrow * kFRows + wv * 16 + c16;  // this lane's row
  const bool rv = r < RT;
  const int t = rv ? static_cast<int>(static_cast<uint32_t>(r) / static_cast<uint32_t>(H)) : 0;
  const int h = rv ? r - t * H : 0;
  const int64_t bt = static_cast<int64_t>(b) * a.T + t;

  // the row's sources: blocks [0, nb), window entries [w0, w1)
  int nb = 0, w0 = 0, w1 = 0;
  if (rv) {
    nb = a.vis ? static_cast<int>(min<int64_t>(max(a.vis[bt], 0), a.S)) : static_cast<int>(a.S);
    w0 = a.wstart ? static_cast<int>(min<int64_t>(max(a.wstart[bt], 0), a.Wt)) : 0;
    w1 = w0 + (a.wlen ? static_cast<int>(min<int64_t>(max(a.wlen[bt], 0), a.Wt - w0)) : static_cast<int>(a.Wt) - w0);
  }
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
  for (int w = 0; w < kFThreads / 64; ++w) {
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

  // queries as the B operand of S^T = K Q^T: lane (row c16) holds dims 32 ks + 8 g .. + 7
  fbf16x8_t qb[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (rv) v = *reinterpret_cast<const uint4*>(a.q + (static_cast<int64_t>(b) * RT + r) * kFD + 32 * ks + 8 * g);
    qb[ks] = __builtin_bit_cast(fbf16x8_t, v);
  }

  // LDS byte offsets, fixed per lane.  Staging: thread tid moves chunk tid % 16 of keys
  // tid / 16 + 16 c.  Row-chunk reads: key 16 kb + c16, logical chunk 4 ks + g.  Transpose reads:
  // key 32 kc + 4 g + c16 / 4 (+16), dims 16 n8 + 4 (c16 % 4) .. + 3.
  const int st_key = tid >> 4;
  const int st_off = st_key * kRowBytes + (((tid & 15) ^ chunk_swizzle(st_key)) << 4);
  int soff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) soff[ks] = c16 * kRowBytes + (((4 * ks + g) ^ chunk_swizzle(c16)) << 4);
  const int tr_key = 4 * g + (c16 >> 2);
  int toff[8];
#pragma unroll
  for (int n8 = 0; n8 < 8; ++n8)
    toff[n8] = tr_key * kRowBytes + (((2 * n8 + ((c16 >> 1) & 1)) ^ chunk_swizzle(tr_key)) << 4) + 8 * (c16 & 1);

  const uint8_t* kseq = reinterpret_cast<const uint8_t*>(a.kblk + static_cast<int64_t>(b) * a.S * kFD);
  const uint8_t* wseq = reinterpret_cast<const uint8_t*>(a.win + static_cast<int64_t>(b) * a.Wt * kFD);
  int voff[kChunks];  // thread tid's 16-byte chunks of a tile: bytes 16 tid + 4096 c
#pragma unroll
  for (int c = 0; c < kChunks; ++c) voff[c] = 16 * tid + 16 * kRowBytes * c;
  // tile it: keys [base, base + TILE) of the blocks (it < n_bt) or of the window, read through a
  // buffer resource whose range ends at the workgroup's last source, so that the rows past it
  // read as zero (never attended) without a branch or an access
  auto load_tile = [&](int it, uint4 (&v)[kChunks]) {
    const bool blk = it < n_bt;
    const int base = blk ? it * kFTile : wlo + (it - n_bt) * kFTile;
    const int lim = blk ? gmax : whi;
    const uint8_t* src = (blk ? kseq : wseq) + static_cast<int64_t>(base) * kRowBytes;
    const int n_bytes = min(lim - base, kFTile) * kRowBytes;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), 0, n_bytes, kBufWord3);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) v[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff[c], 0, 0));
  };
  auto store_tile = [&](int buf, const uint4 (&v)[kChunks]) {
#pragma unroll
    for (int c = 0; c < kChunks; ++c) *reinterpret_cast<uint4*>(Ls[buf] + st_off + 16 * kRowBytes * c) = v[c];
  };

  // m_run: the row's running maximum in scaled log2 units.  lsum: the row's sum of the bf16 weights
  // fed to the products, as a product with an all-ones operand (every element holds the sum), so
  // the normaliser matches the numerator's weights and needs no lane reduction.
  float m_run = kFNegInf;
  ff32x4_t O[8], lsum = ff32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int n8 = 0; n8 < 8; ++n8) O[n8] = ff32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const fbf16x8_t ones = __builtin_bit_cast(fbf16x8_t, make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u));

  uint4 nv[kChunks];
  if (n_tiles > 0) {
    load_tile(0, nv);
    store_tile(0, nv);
  }
  // every load issued so far (queries, first tile) has landed: without this wait the loop's first
  // matrix instruction would wait for the next tile's loads on every iteration
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // one tile; the buffer index is a compile-time constant so that LDS offsets are immediates
  auto step = [&](int it, auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;
    if (it + 1 < n_tiles) load_tile(it + 1, nv);  // in flight during this tile's matrix work
    const uint8_t* lt = Ls[buf];

    // S^T for keys 16 kb + 4 g + i of this tile, rows c16
    constexpr int KB = kFTile / 16;
    ff32x4_t s[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      uint4 kv[4];  // the 16 keys' row chunks, all read before the first product
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kv[ks] = *reinterpret_cast<const uint4*>(lt + 16 * kRowBytes * kb + soff[ks]);
      s[kb] = ff32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(fbf16x8_t, kv[ks]), qb[ks], s[kb], 0, 0, 0);
    }
    // masks (only where some row of the workgroup does not see the whole tile)
    const bool blk_tile = it < n_bt;
    const int base = blk_tile ? it * kFTile : wlo + (it - n_bt) * kFTile;
    float tmax = kFNegInf;
    if (blk_tile && base + kFTile <= nbmin) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, s[kb][i]);
    } else {
      const int lo = (blk_tile ? 0 : w0) - base, hi = (blk_tile ? nb : w1) - base;  // this row's keys of the tile
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int k = 16 * kb + 4 * g + i;
          s[kb][i] = (k >= lo && k < hi) ? s[kb][i] : kFNegInf;
          tmax = fmaxf(tmax, s[kb][i]);
        }
    }
    tmax = fmaxf(tmax, xor_lane<16>(tmax));
    tmax = fmaxf(tmax, xor_lane<32>(tmax));
    const float mt = tmax * a.scale2;
    if (__builtin_amdgcn_ballot_w64(mt > m_run)) {  // some row's maximum moved up
      const float m_new = fmaxf(m_run, mt);
      const float alpha = m_new == kFNegInf ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      lsum *= alpha;
#pragma unroll
      for (int n8 = 0; n8 < 8; ++n8) O[n8] *= alpha;
      m_run = m_new;
    }
    const float nm = m_run == kFNegInf ? 0.0f : -m_run;
    float sv[4 * KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[4 * kb + i] = __builtin_amdgcn_exp2f(fmaf(s[kb][i], a.scale2, nm));
    // O^T[dims 16 n8 + 4 g + i][row c16] += V^T P^T per 32-key chunk; the reduction index runs over
    // keys {4g..4g+3, 16+4g..16+4g+3} of the chunk for lane group g, in both operands
#pragma unroll
    for (int kc = 0; kc < kFTile / 32; ++kc) {
      const fbf16x8_t pb = __builtin_bit_cast(
          fbf16x8_t, make_uint4(pack_bf16x2(sv[8 * kc + 0], sv[8 * kc + 1]), pack_bf16x2(sv[8 * kc + 2], sv[8 * kc + 3]),
                                pack_bf16x2(sv[8 * kc + 4], sv[8 * kc + 5]), pack_bf16x2(sv[8 * kc + 6], sv[8 * kc + 7])));
      lsum = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb, lsum, 0, 0, 0);
      fbf16x8_t va[8];  // the chunk's V^T operands, all read before the first product
#pragma unroll
      for (int n8 = 0; n8 < 8; ++n8) {
        const uint8_t* p = lt + 32 * kRowBytes * kc + toff[n8];
        const fi16x4_t lo = lds_read_tr16(p);
        const fi16x4_t hi = lds_read_tr16(p + 16 * kRowBytes);
        va[n8] = __builtin_bit_cast(fbf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int n8 = 0; n8 < 8; ++n8) O[n8] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[n8], pb, O[n8], 0, 0, 0);
    }
    // the other buffer was last read before the previous barrier
    if (it + 1 < n_tiles) store_tile(buf ^ 1, nv);
    __syncthreads();
  };
#pragma unroll 1
  for (int it = 0; it < n_tiles; it += 2) {
    step(it, IntC<0>{});
    if (it + 1 < n_tiles) step(it + 1, IntC<1>{});
  }

  // the sink, counted once: out = O / (l + e^{sink - m}) with m = max(m_run, sink)
  const float l_run = lsum[0];
  if (!rv) return;
  const float sk = a.sink[h] * kLog2e;
  const float mf = fmaxf(m_run, sk);
  const float fo = m_run == kFNegInf ? 0.0f : exp2f(m_run - mf);
  const float L = fmaf(l_run, fo, exp2f(sk - mf));
  const float rs = fo / L;
  uint16_t* orow = a.out + (static_cast<int64_t>(b) * RT + r) * kFD;  // r < RT here
#pragma unroll
  for (int n8 = 0; n8 < 8; ++n8) {
    const uint2 v = make_uint2(pack_bf16x2(O[n8][0] * rs, O[n8][1] * rs), pack_bf16x2(O[n8][2] * rs, O[n8][3] * rs));
    *reinterpret_cast<uint2*>(orow + 16 * n8 + 4 * g) = v;
  }
}

}  // namespace

size_t hca_prefill_flash_workspace(int64_t B, int64_t S) {
  return align_up(static_cast<size_t>(B) * static_cast<size_t>(S) * kFD * 2, 256);
}

bool hca_prefill_flash_supported(int64_t H, int64_t D) { return D == kFD && H >= 1; }

int launch_hca_prefill_flash(const void* q, const void* kblk, const void* window, const int32_t* vis,
                             const int32_t* wstart, const int32_t* wlen, const float* sink, int64_t B, int64_t T,
                             int64_t H, int64_t S, int64_t Wt, float softmax_scale, void* out, hipStream_t st,
                             const char* who) {
  const int64_t RT = T * H;
  const int64_t gx = ceil_div(RT, kFRows);
  if (gx * B > 0x7fffffff || RT > 0x7fffffff - kFRows) return fail(AEKV_ERR_UNSUPPORTED, "%s: grid too large", who);
  if (S > 0x7fffffff - kFTile || Wt > 0x7fffffff - kFTile)
    return fail(AEKV_ERR_UNSUPPORTED, "%s: %lld blocks / %lld window entries exceed the int32 indexing", who,
                (long long)S, (long long)Wt);
  if (RT == 0 || B == 0) return AEKV_OK;
  FlashArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.kblk = static_cast<const uint16_t*>(kblk);
  a.win = static_cast<const uint16_t*>(window);
  a.vis = vis;
  a.wstart = wstart;
  a.wlen = wlen;
  a.sink = sink;
  a.T = static_cast<int>(T);
  a.S = S;
  a.Wt = Wt;
  a.H = static_cast<int>(H);
  a.scale2 = softmax_scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  a.gx = static_cast<uint32_t>(gx);
  hipLaunchKernelGGL(hca_prefill_flash_kernel, dim3(static_cast<uint32_t>(gx * B)), dim3(kFThreads), 0, st, a);
  return check_launch(who);
}

}  // namespace aekv
