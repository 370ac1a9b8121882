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
//
// The row body (attend_row) is shared by the attention kernel (selection read from global memory)
// and the fused CSA decode kernel (selection left in LDS by the select phase).
#pragma once

#include "tq_device.h"

namespace aekv {
namespace qattn {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kD = 128;
constexpr int kGroup = 32;                    // sources per wave step
constexpr int kSplitSrc = 1024;               // most sources per workgroup (a row is split beyond)
constexpr int64_t kMinSplitSrc = 512;         // fewest sources per split piece
constexpr int64_t kTargetWG = 512;            // split rows until the grid has this many workgroups
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
  float* part;            // [B, n_split, H, kPartStride] (split runs only)
  uint16_t* out;          // [B, H, 128] bf16
};

// Floats per row of the merge buffer: the 4-float pad puts head h's row at bank 4h, so the 16 heads
// of one store or load instruction cover all 64 banks.
constexpr int kObStride = kD + 4;
// Floats per split result of one (row, head): max, sum, two pad, O[128] (16-byte aligned O).
constexpr int kPartStride = kD + 4;

// LDS layout (bytes) for NW waves: wave outputs for the merge | wave stats | per-head factors |
// block ids | WROWS window rows of 256 bytes (the fused decode kernel stages the window there)
template <int NW, int WROWS = 0>
struct QLay {
  static constexpr size_t ob = 0;
  static constexpr size_t st = ob + sizeof(float) * NW * 16 * kObStride;
  static constexpr size_t inv = st + sizeof(float) * NW * 16 * 2;
  static constexpr size_t idx = inv + sizeof(float) * 16;
  static constexpr size_t win = idx + sizeof(int32_t) * kSplitSrc;
  static constexpr size_t bytes = win + sizeof(uint16_t) * kD * WROWS;
};

// Window rows in LDS: the 16-byte chunk j of row r sits at chunk j ^ (r & 15) of the row, so the 16
// rows a lane group reads in one instruction fall on distinct banks.
__device__ __forceinline__ int win_chunk(int r, int j) { return j ^ (r & 15); }

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

// A row's sources: n_comp compressed blocks, then wl window entries from w0 of its cache row cb;
// this workgroup takes [src0, src1).
struct RowSources {
  int64_t cb, n_comp, w0, wl, src0, src1;
};

// The workgroup's selected block ids (entry i of its piece in thread i % (64 NW), slot i / (64 NW)).
template <int NW>
struct RowSel {
  int64_t v[kSplitSrc / (64 * NW)];
};

// A row's raw per-row counts (visible blocks, window start and length), as loaded.
struct RowCounts {
  int32_t vis, ws, wl;
};

// The row's loads that set its sources: the per-row counts and the selected block ids of the
// workgroup's piece (which do not depend on the counts).  Only requests: the caller issues its
// other first-round loads before anything reads these (attend_ranges), so that one memory round
// covers them all (vector loads complete in order, and a count used early, or a load under a
// branch, is waited for before the later requests are issued).  The id loads are unconditional,
// through a buffer resource over the piece's ids (past it, or without a selection: 0 without a
// memory access); store_sel reads only ids below the row's selected count, which lie in the piece.
// (absent counts: all n_comp blocks, window from 0 to its end)
template <int NW>
__device__ __forceinline__ void attend_requests(const QAttnMfmaArgs& a, const int64_t b, const int split,
                                                RowCounts& c, RowSel<NW>& sv) {
  constexpr int kT = 64 * NW;
  // scalar loads (b is uniform; through the constant address space): a vector load of a uniform
  // value is moved to a scalar register right where it is loaded, which waits for it there
  auto count = [&](const int32_t* p, int32_t dflt) {
    const int32_t v = *(const __attribute__((address_space(4))) int32_t*)(p ? p + b : reinterpret_cast<const int32_t*>(a.q));
    return p ? v : dflt;
  };
  c.vis = count(a.vis, 0x7fffffff);
  c.ws = count(a.wstart, 0);
  c.wl = count(a.wlen, 0x7fffffff);
  const int64_t src0 = static_cast<int64_t>(split) * a.split_src;
  const int64_t rest = a.sel ? a.K - src0 : 0;
  const int n_piece = static_cast<int>(rest < a.split_src ? rest : a.split_src);  // <= kSplitSrc
  const __amdgpu_buffer_rsrc_t ids = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int64_t*>(a.sel ? a.sel + b * a.K + src0 : a.sel), 0, n_piece > 0 ? 8 * n_piece : 0, 0x00020000);
#pragma unroll
  for (int j = 0; j < kSplitSrc / kT; ++j) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(ids, (threadIdx.x + j * kT) * 8u, 0, 0);
    sv.v[j] = static_cast<int64_t>((static_cast<uint64_t>(v[1]) << 32) | v[0]);
  }
}

// The row's source ranges from its counts.  Integer clamps (min<int64_t> lowers through doubles).
__device__ __forceinline__ RowSources attend_ranges(const QAttnMfmaArgs& a, const int64_t b, const int split,
                                                    const RowCounts& c) {
  auto clamp = [](int64_t x, int64_t hi) { return x <= 0 ? int64_t{0} : (x < hi ? x : hi); };
  RowSources r;
  r.cb = static_cast<uint32_t>(b) / static_cast<uint32_t>(a.T);  // (32-bit: b < 65536, 1 <= T)
  r.n_comp = clamp(c.vis, a.n_comp);
  r.w0 = clamp(c.ws, a.Wt);
  r.wl = clamp(c.wl, a.Wt - r.w0);
  r.src0 = static_cast<int64_t>(split) * a.split_src;
  const int64_t end = r.src0 + a.split_src;
  r.src1 = r.n_comp + r.wl < end ? r.n_comp + r.wl : end;
  return r;
}

// The selected block ids of [src0, min(src1, n_comp)) into LDS (-1: skipped), read after the next
// barrier.
template <int NW>
__device__ __forceinline__ void store_sel(const QAttnMfmaArgs& a, const RowSources& r, const RowSel<NW>& sv,
                                          unsigned char* lds) {
  constexpr int kT = 64 * NW;
  int32_t* sidx = reinterpret_cast<int32_t*>(lds + QLay<NW>::idx);
  const int64_t nsel = min<int64_t>(r.src1, r.n_comp) - r.src0;
#pragma unroll
  for (int j = 0; j < kSplitSrc / kT; ++j) {
    const int64_t i = threadIdx.x + static_cast<int64_t>(j) * kT;
    const int64_t blk = sv.v[j];
    if (i < nsel) sidx[i] = blk >= 0 && blk < a.S ? static_cast<int32_t>(blk) : -1;
  }
}


// Per-lane constants of a row, independent of its sources: the diagonal's sign bits, the query
// fragments, the H64 operand of the dequantise and the V selectors.
template <int BITS>
struct AttnFrags {
  uint32_t dsign[4][4];
  bf16x8_t qb[4];
  i32x4_t hA[4];
  bf16x8_t esel[2];
  float sink;  // the sink of head threadIdx.x / 8 (threads below 8H; 0 for a split of several)
  uint64_t neg[2];  // the diagonal's sign bits: bit d of neg[d >> 6] (wave-uniform)
};

// The prologue's loads: two entries of the diagonal (dims lane and 64 + lane; the wave's ballots
// of their signs give every lane the signs of its own dims), the query row of the lane's head, and
// the sink the merge needs at the end (requested here so that the merge does not wait for it).
// Each load instruction of a wave costs the CU's memory pipeline time per lane, so the diagonal
// is not read as 32 dims per lane.
struct PrologueRaw {
  float dv[2];
  uint4 qw[4];
  float sink;
};

// A bf16 row of kD dims held by the lane pair l, l ^ 16 (lane groups g, g ^ 1: one 16-lane column)
// as one 16-byte piece per lane and k-step: dims 16 (2 ks + (g & 1)) + 8 (g >> 1) + 0..7.  The
// operands want, per lane, dims 32 ks + 4 g + 0..3 (lo) and 32 ks + 16 + 4 g + 0..3 (hi); a lane's
// piece holds its own lo (g even) or hi (g odd) and its partner's other half, so one
// permlane16_swap per dword pair (odd rows of the first operand swapped with even rows of the
// second) hands each half to its lane.  Both lanes of a pair must run it.  Loading 16-byte pieces
// halves the load instructions of a row (each one a pass through the CU's address unit).
__device__ __forceinline__ int pair_piece_dims(int g) { return 16 * (g & 1) + 8 * (g >> 1); }

__device__ __forceinline__ void pair_halves(const uint4& p, uint2& lo, uint2& hi) {
  const auto sx = __builtin_amdgcn_permlane16_swap(p.x, p.z, false, false);
  const auto sy = __builtin_amdgcn_permlane16_swap(p.y, p.w, false, false);
  const uint32_t lx = sx[0], hx = sx[1], ly = sy[0], hy = sy[1];  // (elements copied out first)
  lo = make_uint2(lx, ly);
  hi = make_uint2(hx, hy);
}

__device__ __forceinline__ void prologue_loads(const QAttnMfmaArgs& a, const int64_t b, PrologueRaw& r) {
  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
  // The lane's 32 dims, for every key it holds: element j of k-step ks (bf16x8) is dim
  // 16*(2ks + (j >> 2)) + 4g + (j & 3); the query row of head c16 arrives as pair pieces
  // (pair_halves).  Every load (the diagonal, the query row) is issued before any is used: one
  // memory round.  Lanes past the heads read head 0's row and use zeros.
  const uint16_t* qr = a.q + (b * a.H + (c16 < a.H ? c16 : 0)) * kD + pair_piece_dims(g);
  r.dv[0] = a.diag[lane];
  r.dv[1] = a.diag[64 + lane];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) r.qw[ks] = *reinterpret_cast<const uint4*>(qr + 32 * ks);
  const int th = static_cast<int>(threadIdx.x >> 3) < a.H ? static_cast<int>(threadIdx.x >> 3) : 0;
  r.sink = a.n_split == 1 ? a.sink[th] : 0.0f;
}

template <int BITS>
__device__ __forceinline__ void prologue_build(const QAttnMfmaArgs& a, const PrologueRaw& r, AttnFrags<BITS>& f) {
  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
  const bool has_head = c16 < a.H;
  uint2 lo[4], hi[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) pair_halves(r.qw[ks], lo[ks], hi[ks]);
  f.sink = r.sink;
  // dsign: the diagonal's sign bits for the lane's dims, per packed bf16 pair (dword e of k-step
  // ks), from the signs of all 128 dims (bit d of neg[d >> 6], every lane of the wave active)
  const uint64_t neg[2] = {__builtin_amdgcn_ballot_w64(r.dv[0] < 0.0f), __builtin_amdgcn_ballot_w64(r.dv[1] < 0.0f)};
  f.neg[0] = neg[0];
  f.neg[1] = neg[1];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int hv = 0; hv < 2; ++hv) {
      const uint32_t nb = static_cast<uint32_t>(neg[ks >> 1] >> ((32 * (ks & 1) + 16 * hv + 4 * g) & 63));  // dims 0..3 of the four
      f.dsign[ks][2 * hv] = ((nb & 1u) ? 0x8000u : 0u) | ((nb & 2u) ? 0x80000000u : 0u);
      f.dsign[ks][2 * hv + 1] = ((nb & 4u) ? 0x8000u : 0u) | ((nb & 8u) ? 0x80000000u : 0u);
    }
  // queries (times the diagonal) as the B operand of S^T: lane (head c16), the lane's dims
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const uint4 w = make_uint4(lo[ks].x ^ f.dsign[ks][0], lo[ks].y ^ f.dsign[ks][1], hi[ks].x ^ f.dsign[ks][2],
                               hi[ks].y ^ f.dsign[ks][3]);
    f.qb[ks] = __builtin_bit_cast(bf16x8_t, has_head ? w : make_uint4(0u, 0u, 0u, 0u));
  }
  // H64 rows 16a + c16 as int8 +-1 over the lane's code indices (the A operand of the dequantise).
  // Byte `by` of dword dw holds H64[16a + c16][c] = (-1)^parity((16a + c16) & c) for the code index
  // c = code_index(g, 4dw + by); the bits of c split into disjoint fields (g | dw | by for 8-bit,
  // g | dw >> 1 | by | dw & 1 for 4-bit), so the parity is parity(a & g) ^ X(dw) ^ parity(mb & by)
  // with per-lane X and mb, and each dword is one xor of masks.
  const uint32_t mb = BITS == 8 ? (c16 & 3) : ((c16 >> 1) & 3);
  uint32_t m0 = 0u;  // 0xFF in the bytes by with parity(mb & by) = 1
#pragma unroll
  for (int by = 1; by < 4; ++by) m0 |= (__builtin_popcount(mb & by) & 1) ? (0xFFu << (8 * by)) : 0u;
#pragma unroll
  for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
    for (int dw = 0; dw < 4; ++dw) {
      const int xd = BITS == 8 ? __builtin_popcount((c16 >> 2) & dw) : __builtin_popcount(c16 & (8 * (dw >> 1) + (dw & 1)));
      const uint32_t neg = m0 ^ (((xd ^ __builtin_popcount(a4 & g)) & 1) ? 0xFFFFFFFFu : 0u);
      f.hA[a4][dw] = static_cast<int>(0x01010101u ^ (neg & 0xFEFEFEFEu));
    }
  // 0/1 selectors: esel[h] (lane column c16, element j of group g) = 1 iff g == c16 >> 2 and
  // j == (c16 & 3) + 4h, i.e. column c16 picks dim 16*(2ks + h) + c16 of k-step ks
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j0 = 2 * e;
      const bool mine = g == (c16 >> 2);
      w[e] = (mine && j0 == (c16 & 3) + 4 * h ? 0x3F80u : 0u) | (mine && j0 + 1 == (c16 & 3) + 4 * h ? 0x3F800000u : 0u);
    }
    f.esel[h] = __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
  }
}

// ---- one 32-source group of a wave: its rows requested, then decoded and attended -------------
// A group is two blocks of 16 keys; lane (key c16 of block kb) holds its source's row: a code row
// (kind 1, block id blk of cache row cb), a window row (kind 2, entry wrow) or nothing (kind 0).
// WIN: the group may hold window rows (kind 2); without, it holds code rows only.
template <int BITS, bool WIN = true>
struct GroupIn {
  int kind[2];
  uint32_t cw[2][2][BITS == 8 ? 4 : 2];
  float sraw[2];
  uint4 wq[WIN ? 2 : 1][4];  // window rows as pair pieces (pair_halves)
};

// The lane's source of block kb: kind and block id (kind 1) or window entry (kind 2).
struct SrcRef {
  int kind;
  int64_t at;
};

// Requests the rows of both blocks (every load issued before any is used).  win_lds (nullable):
// the cache row's window entries staged in LDS (win_chunk layout) instead of global memory.
template <int BITS, bool WIN = true>
__device__ __forceinline__ void group_fetch(const QAttnMfmaArgs& a, const int64_t cb, const SrcRef (&src)[2],
                                            const unsigned char* win_lds, GroupIn<BITS, WIN>& in) {
  constexpr int RB = BITS == 8 ? kD : kD / 2;   // code bytes per row
  constexpr int HB = RB / 2;                    // code bytes per 64-code half
  const int lane = threadIdx.x & 63, g = lane >> 4;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    in.kind[kb] = src[kb].kind;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int e = 0; e < (BITS == 8 ? 4 : 2); ++e) in.cw[kb][hh][e] = 0u;
    in.sraw[kb] = 0.0f;
    if (src[kb].kind == 1) {
      const int64_t blk = src[kb].at;
      const uint8_t* row = a.codes + (cb * a.S + blk) * RB;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        if constexpr (BITS == 8) {
          const uint4 v = *reinterpret_cast<const uint4*>(row + HB * hh + 16 * g);
          in.cw[kb][hh][0] = v.x;
          in.cw[kb][hh][1] = v.y;
          in.cw[kb][hh][2] = v.z;
          in.cw[kb][hh][3] = v.w;
        } else {
          const uint2 v = *reinterpret_cast<const uint2*>(row + HB * hh + 8 * g);
          in.cw[kb][hh][0] = v.x;
          in.cw[kb][hh][1] = v.y;
        }
      }
      in.sraw[kb] = a.scale[cb * a.S + blk];
    }
    if (WIN && src[kb].kind == 2) {
      const int64_t wrow = src[kb].at;
      if (win_lds) {
        // the pair piece of k-step ks, dims 16 (2ks + (g & 1)) + 8 (g >> 1): 16-byte chunk
        // 4ks + 2 (g & 1) + (g >> 1) of the row
        const int r = static_cast<int>(wrow);
        const unsigned char* rp = win_lds + 2 * kD * r;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          in.wq[WIN ? kb : 0][ks] =
              *reinterpret_cast<const uint4*>(rp + 16 * win_chunk(r, 4 * ks + 2 * (g & 1) + (g >> 1)));
      } else {
        const uint16_t* wr = a.win + (cb * a.Wt + wrow) * kD + pair_piece_dims(g);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) in.wq[WIN ? kb : 0][ks] = *reinterpret_cast<const uint4*>(wr + 32 * ks);
      }
    }
  }
}

constexpr uint32_t kPastRange = 0x80000000u; // an offset past every range (ranges are < 2^31 bytes)

// Window entry e (< Wt, else no source) of decode row b as block 0 of lane column c16's group
// (block 1 empty), its row as pair pieces, through a buffer resource over the row's Wt entries: the
// loads are unconditional (a branch around them would make the compiler copy their registers, and
// so wait for them, where the branch joins) and an entry past Wt reads zeros without a memory
// access.  Rows of Wt * kD * 2 < 2^31 bytes.
template <int BITS>
__device__ __forceinline__ void window_fetch(const QAttnMfmaArgs& a, const int64_t b, const int e, GroupIn<BITS>& in) {
  const int g = (threadIdx.x & 63) >> 4;
  const bool ok = e < a.Wt;
  in.kind[0] = ok ? 2 : 0;
  in.kind[1] = 0;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int i = 0; i < (BITS == 8 ? 4 : 2); ++i) in.cw[kb][hh][i] = 0u;
    in.sraw[kb] = 0.0f;
  }
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.win + b * a.Wt * kD), 0, static_cast<int>(a.Wt * kD * 2), 0x00020000);
  const uint32_t o = ok ? static_cast<uint32_t>(e) * (2 * kD) + 2 * pair_piece_dims(g) : kPastRange;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, o + 64 * ks, 0, 0);
    in.wq[0][ks] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

// Online-softmax state and output of head c16 (replicated over the four lane groups).
struct AttnState {
  float m_run, l_run;
  f32x4_t O[8];
};

__device__ __forceinline__ void attn_state_init(AttnState& s) {
  s.m_run = kNegInf;
  s.l_run = 0.0f;
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) s.O[nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
}

// Decodes the group's rows and folds its 32 sources into the state.
// ok_mask (per block kb, nullable): a per-lane validity on top of the row kinds, e.g. whether the
// lane's candidate made the selection.
template <int BITS, bool WIN = true>
__device__ __forceinline__ void group_consume(const QAttnMfmaArgs& a, const AttnFrags<BITS>& f,
                                              const GroupIn<BITS, WIN>& in, AttnState& s,
                                              const bool* ok_mask = nullptr) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const uint32_t (&dsign)[4][4] = f.dsign;
  const bf16x8_t (&qb)[4] = f.qb;
  const i32x4_t (&hA)[4] = f.hA;
  const bf16x8_t (&esel)[2] = f.esel;
  const int (&kind)[2] = in.kind;
  const auto& cw = in.cw;
  const float (&sraw)[2] = in.sraw;
  const auto& wq = in.wq;
  // a group with no source at all (past the end of a piece) changes nothing
  if (__builtin_amdgcn_ballot_w64(kind[0] != 0 || kind[1] != 0) == 0) return;
  const float kscale_unit = (BITS == 4 ? 1.0f / 16.0f : 1.0f) * a.wscale;
  bf16x8_t kf[2][4];
  bool okk[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    okk[kb] = kind[kb] != 0 && (!ok_mask || ok_mask[kb]);
    const float fk = sraw[kb] * kscale_unit;  // 0 for lanes without a code row (no scale loaded)
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
      if (WIN && kind[kb] == 2) {
        constexpr int kw = 0;  // (wq has one block without window rows)
        const int wb = WIN ? kb : kw;
        // (the lane pair of a window row shares its kind: kinds depend on the column c16 only)
        uint2 lo, hi;
        pair_halves(wq[wb][ks], lo, hi);
        w4[0] = lo.x ^ dsign[ks][0];
        w4[1] = lo.y ^ dsign[ks][1];
        w4[2] = hi.x ^ dsign[ks][2];
        w4[3] = hi.y ^ dsign[ks][3];
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
    const float mnew = fmaxf(s.m_run, tm);
    const float corr = s.m_run == kNegInf ? 0.0f : __expf(s.m_run - mnew);
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
    s.l_run = s.l_run * corr + ps;
    // O is rescaled only when some head's running max moved (corr is exactly 1 otherwise, and O is
    // still 0 while the max is -inf): most groups skip the 32 multiplies
    if (__builtin_amdgcn_ballot_w64(mnew != s.m_run && s.m_run != kNegInf) != 0) {
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) s.O[nb] *= corr;
    }
    s.m_run = mnew;
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
    s.O[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, s.O[nb], 0, 0, 0);
  }
}

// Merges the NW waves' states (and the sink, unless this is one split of several) and writes the
// row's output, or its split result (max, sum, O) for the combine.  sink_h: the sink of head
// threadIdx.x / 8, requested with the prologue (AttnFrags::sink); neg: the diagonal's sign bits
// (AttnFrags::neg), so that the diagonal comes off the output without a memory round.
template <int NW>
__device__ __forceinline__ void attend_finish(const QAttnMfmaArgs& a, const int64_t b, const int split,
                                              unsigned char* lds, const AttnState& s, const float sink_h,
                                              const uint64_t (&neg)[2]) {
  constexpr int kW = NW, kT = 64 * NW;
  using L = QLay<NW>;
  float* Ob = reinterpret_cast<float*>(lds + L::ob);    // [wave][head][kObStride]
  float* stat = reinterpret_cast<float*>(lds + L::st);  // [wave][head][m, l]
  float* inv = reinterpret_cast<float*>(lds + L::inv);  // [head]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  const int H = a.H;
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
    *reinterpret_cast<f32x4_t*>(Ob + (wv * 16 + c16) * kObStride + 16 * nb + 4 * g) = s.O[nb];
  if (g == 0) {
    stat[(wv * 16 + c16) * 2] = s.m_run;
    stat[(wv * 16 + c16) * 2 + 1] = s.l_run;
  }
  __syncthreads();
  // per head: M = max(sink, wave maxima), the waves' factors e^{m_w - M}, and the normaliser L;
  // the factors replace the maxima in stat, 1/L (or L for a split) is kept aside.  Thread 8h + w of
  // the first two waves takes head h and wave w, and the 8 lanes of a head reduce by lane exchanges.
  if (threadIdx.x < 128) {  // wave-uniform
    const int h = threadIdx.x >> 3, w = threadIdx.x & 7;
    const bool valid = h < H && w < kW;
    const float mw = valid ? stat[(w * 16 + h) * 2] : kNegInf;
    const float lw = valid ? stat[(w * 16 + h) * 2 + 1] : 0.0f;
    float M = a.n_split == 1 ? fmaxf(mw, sink_h) : mw;
    M = fmaxf(M, xor_lane<1>(M));
    M = fmaxf(M, xor_lane<2>(M));
    M = fmaxf(M, xor_lane<4>(M));
    const float f = mw == kNegInf ? 0.0f : __expf(mw - M);
    float L = f * lw;
    L += xor_lane<1>(L);
    L += xor_lane<2>(L);
    L += xor_lane<4>(L);
    if (a.n_split == 1) L += __expf(sink_h - M);
    if (valid) stat[(w * 16 + h) * 2] = f;
    if (w == 0 && h < H) {
      if (a.n_split == 1) {
        inv[h] = M == kNegInf ? 0.0f : 1.0f / L;  // no source and sink -inf: 0
      } else {
        float* dst = a.part + ((b * a.n_split + split) * H + h) * kPartStride;
        dst[0] = M;
        dst[1] = L;
      }
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
      const f32x4_t o = *reinterpret_cast<const f32x4_t*>(Ob + (w * 16 + h) * kObStride + d4);
      acc = f32x4_t{fmaf(f, o[0], acc[0]), fmaf(f, o[1], acc[1]), fmaf(f, o[2], acc[2]), fmaf(f, o[3], acc[3])};
    }
    // times the +-1 diagonal: a sign flip of dims d4 .. d4 + 3 (exact)
    // (a select, not an index: a runtime index into the array would put the fragments in scratch)
    const uint32_t sg = static_cast<uint32_t>((d4 < 64 ? neg[0] : neg[1]) >> (d4 & 63));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = acc[e];  // (a bit cast of the vector element itself would read element 0)
      acc[e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) ^ (((sg >> e) & 1u) << 31));
    }
    if (a.n_split == 1) {
      const float r = inv[h];
      const uint2 v = make_uint2(pack_bf16x2(acc[0] * r, acc[1] * r), pack_bf16x2(acc[2] * r, acc[3] * r));
      *reinterpret_cast<uint2*>(a.out + (b * H + h) * kD + d4) = v;
    } else {
      *reinterpret_cast<f32x4_t*>(a.part + ((b * a.n_split + split) * H + h) * kPartStride + 4 + d4) = acc;
    }
  }
}

// The row's attention over its sources (after attend_ranges and the prologue's loads).  The query
// fragments are built from praw once the wave's first group's rows are requested, so that the
// gather does not wait for them.  win_lds (nullable): the cache row's window entries 0 .. Wt-1
// staged in LDS (win_chunk layout) instead of read from global memory.  PIPE: a wave requests its
// next group's rows before decoding the current one (the 4-wave prefill instance, whose register
// budget has room for them).
template <int BITS, int NW, bool PIPE = false>
__device__ __forceinline__ void attend_main(const QAttnMfmaArgs& a, const int64_t b, const int split,
                                            unsigned char* lds, const PrologueRaw& praw, const RowSources& rs,
                                            const unsigned char* win_lds) {
  constexpr int kW = NW;
  using L = QLay<NW>;
  const int32_t* sidx = reinterpret_cast<const int32_t*>(lds + L::idx);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c16 = lane & 15;
  const int64_t cb = rs.cb, n_comp = rs.n_comp, w0 = rs.w0, src0 = rs.src0, src1 = rs.src1;
  __syncthreads();  // sidx

  AttnState s;
  attn_state_init(s);
  const int n_groups = src1 > src0 ? static_cast<int>((src1 - src0 + kGroup - 1) / kGroup) : 0;
  // group G's sources (32 per group): both blocks' rows are requested before either is decoded
  auto fetch = [&](const int G, GroupIn<BITS>& in) {
    SrcRef src[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      // lane (key c16 of block kb): its source, code bytes (two halves) or window dims
      const int64_t si = src0 + static_cast<int64_t>(G) * kGroup + 16 * kb + c16;
      src[kb].kind = 0;
      src[kb].at = -1;
      if (si < n_comp) {
        const int64_t blk = a.sel ? sidx[si - src0] : si;
        src[kb].kind = blk >= 0 ? 1 : 0;
        src[kb].at = blk;
      } else if (si < src1) {
        src[kb].kind = 2;
        src[kb].at = w0 + (si - n_comp);
      }
    }
    group_fetch<BITS>(a, cb, src, win_lds, in);
  };
  AttnFrags<BITS> f;
  if constexpr (PIPE) {
    // the next group's rows are requested before this group is decoded
    GroupIn<BITS> cur, nxt;
    if (wv < n_groups) fetch(wv, cur);
    __builtin_amdgcn_sched_barrier(0);
    prologue_build<BITS>(a, praw, f);
#pragma unroll 1
    for (int G = wv; G < n_groups; G += kW) {
      const bool more = G + kW < n_groups;  // wave-uniform
      if (more) fetch(G + kW, nxt);
      group_consume<BITS>(a, f, cur, s);
      if (more) cur = nxt;
    }
  } else {
    bool built = false;  // wave-uniform
#pragma unroll 1
    for (int G = wv; G < n_groups; G += kW) {
      GroupIn<BITS> in;
      fetch(G, in);
      if (!built) {
        __builtin_amdgcn_sched_barrier(0);
        prologue_build<BITS>(a, praw, f);
        built = true;
      }
      group_consume<BITS>(a, f, in, s);
    }
    if (!built) prologue_build<BITS>(a, praw, f);  // (a wave without a group)
  }
  // ---- merge the waves (and the sink, unless this is one split of several) ----
  attend_finish<NW>(a, b, split, lds, s, f.sink, f.neg);
}


// attend_requests + prologue_loads + attend_ranges + store_sel + attend_main: the row's counts, its
// selected block ids and the prologue's loads are requested in one memory round.
template <int BITS, int NW>
__device__ __forceinline__ void attend_row(const QAttnMfmaArgs& a, const int64_t b, const int split,
                                           unsigned char* lds) {
  RowSel<NW> sv;
  RowCounts cnt;
  attend_requests<NW>(a, b, split, cnt, sv);
  PrologueRaw praw;
  prologue_loads(a, b, praw);
  __builtin_amdgcn_sched_barrier(0);  // every request above is issued before a count is read
  const RowSources rs = attend_ranges(a, b, split, cnt);
  if (a.sel) store_sel<NW>(a, rs, sv, lds);
  attend_main<BITS, NW, NW == 4>(a, b, split, lds, praw, rs, nullptr);
}

// ---- rows that attend every block, without per-row counts (the decode step's HCA call) ----
// Buffer resources over one cache row's codes, scales and window entries: the hardware checks each
// load's offset against the range and returns zeros past it, so a lane without such a source loads
// at an offset past the range instead of branching.  The loads are buffer intrinsics, which the
// compiler leaves where they are written (it may merge or move plain loads that feed a loop
// variable down to their first use, which undoes a prefetch).
constexpr uint32_t kBufWord3 = 0x00020000u;  // 32-bit data, raw (unswizzled) addressing

struct DenseRsrc {
  __amdgpu_buffer_rsrc_t codes, scale, win;
};

template <int BITS>
__device__ __forceinline__ DenseRsrc dense_rsrc(const QAttnMfmaArgs& a, const int64_t b) {
  constexpr int RB = BITS == 8 ? kD : kD / 2;
  DenseRsrc r;
  r.codes = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.codes + b * a.S * RB), 0,
                                              static_cast<int>(a.S * RB), kBufWord3);
  r.scale = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.scale + b * a.S), 0, static_cast<int>(a.S * 4),
                                              kBufWord3);
  r.win = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.win + b * a.Wt * kD), 0,
                                            static_cast<int>(a.Wt * kD * 2), kBufWord3);
  return r;
}

// A group's rows: every lane issues the same loads (a code row's two halves, its scale and, WIN,
// a window row), at offsets past the range for the sources it does not have, which read as zeros
// (a zero scale, as group_consume expects of a lane without a code row).
template <int BITS, bool WIN>
__device__ __forceinline__ void dense_fetch(const QAttnMfmaArgs& a, const DenseRsrc& rs, const int64_t src0,
                                            const int64_t src1, const int G, GroupIn<BITS, WIN>& in) {
  constexpr int RB = BITS == 8 ? kD : kD / 2;
  constexpr int HB = RB / 2;
  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
  const int64_t n_comp = a.n_comp;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int64_t si = src0 + static_cast<int64_t>(G) * kGroup + 16 * kb + c16;
    const bool is_code = si < n_comp && si < src1;
    const bool is_win = WIN && !is_code && si < src1;
    in.kind[kb] = is_code ? 1 : (is_win ? 2 : 0);
    const uint32_t co = is_code ? static_cast<uint32_t>(si) * RB : kPastRange;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      if constexpr (BITS == 8) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs.codes, co + HB * hh + 16 * g, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) in.cw[kb][hh][e] = v[e];
      } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs.codes, co + HB * hh + 8 * g, 0, 0);
        in.cw[kb][hh][0] = v[0];
        in.cw[kb][hh][1] = v[1];
      }
    }
    in.sraw[kb] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                rs.scale, is_code ? static_cast<uint32_t>(si) * 4 : kPastRange, 0, 0));
    if constexpr (WIN) {
      const uint32_t wo =
          is_win ? static_cast<uint32_t>(si - n_comp) * (2 * kD) + 2 * pair_piece_dims(g) : kPastRange;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs.win, wo + 64 * ks, 0, 0);
        in.wq[kb][ks] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }
}

// One split [src0, src1) of decode row b over every block then every window entry (T = 1, no
// selection, no counts).  The query's and the wave's first group's rows are requested together.
// Without window entries in the split (!WIN), the second group's rows are requested in the same
// round (the registers allow it: 196, two waves per SIMD either way; a wave that waited for the
// query fragments before requesting them could stall on them after its first group) and each group
// is decoded while the group after next is requested (two buffers, no copies).  A split with window
// entries (WIN: 64 more bytes per lane and block) keeps one buffer: a group's successor is
// requested after it is decoded.
template <int BITS, int NW, bool WIN>
__device__ __forceinline__ void attend_dense(const QAttnMfmaArgs& a, const int64_t b, const int split,
                                             unsigned char* lds) {
  constexpr int kW = NW;
  const int wv = threadIdx.x >> 6;
  const int64_t src0 = static_cast<int64_t>(split) * a.split_src;
  const int64_t src1 = min<int64_t>(a.n_comp + a.Wt, src0 + a.split_src);
  const int n_groups = src1 > src0 ? static_cast<int>((src1 - src0 + kGroup - 1) / kGroup) : 0;
  // (the scheduling barriers keep each request batch in program order: a wait counts requests in
  // issue order, so a batch moved behind a later one would make its wait include that one too)
  const DenseRsrc rs = dense_rsrc<BITS>(a, b);
  PrologueRaw praw;
  prologue_loads(a, b, praw);
  __builtin_amdgcn_sched_barrier(0);
  GroupIn<BITS, WIN> in0, in1;
  dense_fetch<BITS, WIN>(a, rs, src0, src1, wv, in0);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!WIN) {
    dense_fetch<BITS, WIN>(a, rs, src0, src1, wv + kW, in1);
    __builtin_amdgcn_sched_barrier(0);
  }
  AttnFrags<BITS> f;
  prologue_build<BITS>(a, praw, f);
  AttnState s;
  attn_state_init(s);
  if constexpr (WIN) {
#pragma unroll 1
    for (int G = wv; G < n_groups; G += kW) {  // wave-uniform
      group_consume<BITS, WIN>(a, f, in0, s);
      dense_fetch<BITS, WIN>(a, rs, src0, src1, G + kW, in0);
    }
  } else {
    // Both buffers are decoded on every pass, so that no load is used only under a branch (the
    // compiler would move it there, after the wait it was meant to overlap).  A group past the split
    // has no sources and changes nothing (all keys masked: the state's factor is exactly 1).
#pragma unroll 1
    for (int G = wv; G < n_groups; G += 2 * kW) {  // wave-uniform
      group_consume<BITS, WIN>(a, f, in0, s);
      __builtin_amdgcn_sched_barrier(0);
      dense_fetch<BITS, WIN>(a, rs, src0, src1, G + 2 * kW, in0);
      __builtin_amdgcn_sched_barrier(0);
      group_consume<BITS, WIN>(a, f, in1, s);
      __builtin_amdgcn_sched_barrier(0);
      dense_fetch<BITS, WIN>(a, rs, src0, src1, G + 3 * kW, in1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  attend_finish<NW>(a, b, split, lds, s, f.sink, f.neg);
}

// One row (or one split of a long row) per workgroup of 64 * NW threads.
//
// Workgroups are dispatched round-robin over the 8 XCDs (linear id L on XCD L % 8), each with its
// own L2.  For prefill rows (T > 1 targets per cache row, rows sequence-major) the linear ids are
// renumbered so that XCD x runs the consecutive range [x n/8, (x+1) n/8) of (row, split) pairs,
// i.e. whole sequences, whose code rows then stay in that XCD's L2 for all of their targets.
template <int BITS, int NW>
__global__ __launch_bounds__(64 * NW) void quant_attn_mfma_kernel(QAttnMfmaArgs a) {
  touch_kernargs<sizeof(a)>();
  extern __shared__ __align__(16) unsigned char lds[];
  int64_t row = blockIdx.y, split = blockIdx.x;
  const uint32_t nx = gridDim.x, n_wg = nx * gridDim.y;
  if (a.T > 1 && n_wg % 8 == 0) {
    const uint32_t L = blockIdx.y * nx + blockIdx.x;
    const uint32_t w = (L % 8) * (n_wg / 8) + L / 8;
    row = w / nx;
    split = w % nx;
  }
  attend_row<BITS, NW>(a, row, static_cast<int>(split), lds);
}

// Decode rows over every block (T = 1, no selection, no counts): attend_dense, one workgroup of
// 512 threads per (split, row).
template <int BITS>
__global__ __launch_bounds__(kThreads) void quant_attn_dense_kernel(QAttnMfmaArgs a) {
  touch_kernargs<sizeof(a)>();
  extern __shared__ __align__(16) unsigned char lds[];
  const int64_t row = blockIdx.y;
  const int split = static_cast<int>(blockIdx.x);
  const bool has_win = static_cast<int64_t>(split + 1) * a.split_src > a.n_comp && a.Wt > 0;  // workgroup-uniform
  if (has_win)
    attend_dense<BITS, kWaves, true>(a, row, split, lds);
  else
    attend_dense<BITS, kWaves, false>(a, row, split, lds);
}

}  // namespace qattn
}  // namespace aekv
