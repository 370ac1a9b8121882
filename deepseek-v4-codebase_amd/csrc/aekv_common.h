// Shared host/device helpers for libaetherkv (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>

#include "aetherkv.h"

namespace aekv {

// ---- host-side error reporting -------------------------------------------------------------
// Stores a thread-local message and returns `status` so call sites can `return fail(...)`.
int fail(int status, const char* fmt, ...);
// Checks hipGetLastError() after a launch; returns AEKV_OK or AEKV_ERR_HIP with a message.
int check_launch(const char* what);

inline bool is_pow2(int64_t d) { return d > 0 && (d & (d - 1)) == 0; }
inline bool is_aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline size_t dtype_size(int dt) { return dt == AEKV_F32 || dt == AEKV_I32 ? 4 : (dt == AEKV_I64 ? 8 : 2); }
inline bool is_float_dtype(int dt) { return dt == AEKV_F32 || dt == AEKV_F16 || dt == AEKV_BF16; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
// fp32(d ** -0.5): the python double d**-0.5 rounded to fp32, as torch does for `out * (d ** -0.5)`.
float wht_scale(int d);
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Matrix-core indexer for quantised keys (csa_indexer_mfma.hip).
bool mfma_indexer_supported(int IH, int IC, int k, int64_t S);
size_t mfma_indexer_workspace(int64_t B, int64_t S, int32_t k);
int launch_mfma_indexer(const float* q, const float* w, const void* codes, const float* kscale, const float* diag,
                        const int32_t* valid, int64_t B, int64_t T, int64_t S, int IH, int IC, int bits, int k,
                        int mode, void* ws, int64_t* out_idx, float* out_score, hipStream_t st, const char* who);
bool use_specialised_codec();
// Host-side argument checks of the quantised-key indexer for B * T rows (csa_indexer.hip).
int validate_quant_rows(const float* index_q, const float* index_weight, const void* key_codes,
                        const float* key_scale, const float* diag, int64_t B, int64_t T, int64_t S, int32_t IH,
                        int32_t IC, int32_t bits, int32_t k, int32_t mode, void* ws, size_t ws_bytes,
                        int64_t* out_idx, const char* who);
// Matrix-core decode attention for head_dim 128 (quant_attn_mfma.hip).
bool quant_attn_mfma_supported(int64_t H, int64_t D);
bool quant_attn_mfma_fits(int64_t rows, int64_t n_src);  // grid and split-combine limits
// Chunked-prefill HCA attention over bf16 blocks [B, S, 128] already decoded (prefill_flash.hip).
bool hca_prefill_flash_supported(int64_t H, int64_t D);
size_t hca_prefill_flash_workspace(int64_t B, int64_t S);  // the decoded blocks
int launch_hca_prefill_flash(const void* q, const void* kblk, const void* window, const int32_t* vis,
                             const int32_t* wstart, const int32_t* wlen, const float* sink, int64_t B, int64_t T,
                             int64_t H, int64_t S, int64_t Wt, float softmax_scale, void* out, hipStream_t st,
                             const char* who);
// Drop-in sink attention on the matrix cores, head_dim 128, bf16/fp16 (sink_attention_mfma.hip):
// q [B, T, H, 128], kv [B, S, 2, 128], per-target indices idx [B, T, K] (idx_kind 4/8: int32/int64)
// or every source (idx_kind 0, K = S).  A workspace (may be null) lets launches with few
// workgroups split the sources; sink_attention_mfma_workspace gives its size (0: no split).
bool sink_attention_mfma_supported(int32_t dtype, int64_t D);
size_t sink_attention_mfma_workspace(bool dense, int64_t B, int64_t T, int64_t H, int64_t S, int64_t K);
int sink_attention_mfma(const void* q, const void* kv, const void* idx, int idx_kind, const void* sink,
                        int sink_scalar, int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t S, int64_t K,
                        float scale, void* ws, size_t ws_bytes, void* out, hipStream_t st, const char* who);
// The flash kernel for dense calls (prefill_flash.hip): 64 (target, head) rows per workgroup, tiles
// of dense_flash_tile() sources; with n_split > 1 each row's tiles are split into n_split pieces
// whose (max, sum, O) go to part (the layout of sink_attention_mfma's combine).
int64_t dense_flash_row_blocks(int64_t T, int64_t H);
int64_t dense_flash_tile();
int launch_dense_flash_attention(const void* q, const void* kv, const void* sink, int sink_scalar, int32_t dtype,
                                 int64_t B, int64_t T, int64_t H, int64_t S, float softmax_scale, int n_split,
                                 float* part, void* out, hipStream_t st, const char* who);
size_t quant_attn_mfma_workspace(int64_t B, int64_t H, int64_t n_src);
// K: the selection's length (sel [rows or B, K]), or with all_blocks the number of blocks taken in
// order, 0 .. K-1, of each row of S (the row stride of codes and scale).
int launch_quant_attn_mfma(const void* q, const void* codes, const float* scale, const int64_t* sel,
                           const void* window, const float* sink, const float* diag, int64_t B, int64_t H, int64_t S,
                           int64_t K, bool all_blocks, int64_t W, int bits, float softmax_scale, void* ws,
                           void* out, hipStream_t st, const char* who);
// Rows are targets (T per cache row) with per-row compressed counts vis and window slices
// [wstart, wstart + wlen) of a [B / T, Wt, 128] window buffer (any of the three may be null).
int launch_quant_attn_mfma_rows(const void* q, const void* codes, const float* scale, const int64_t* sel,
                                const int32_t* vis, const void* window, const int32_t* wstart, const int32_t* wlen,
                                const float* sink, const float* diag, int64_t rows, int64_t T, int64_t H, int64_t S,
                                int64_t K, bool all_blocks, int64_t Wt, int bits, float softmax_scale, void* ws,
                                void* out, hipStream_t st, const char* who);

// ---- device helpers ------------------------------------------------------------------------
// Requests every 64-byte line of the kernel's argument block in one scalar-memory round.  The
// compiler loads an argument where it is first needed, often behind a branch on an argument loaded
// before it, and each such load is a memory round trip of its own while the argument block is not
// cached (a graph replayed over more data than the caches hold); after this call they hit the
// scalar cache.  NBYTES: the size of the kernel's arguments.
template <int NBYTES>
__device__ __forceinline__ void touch_kernargs() {
  typedef const __attribute__((address_space(4))) uint32_t karg_u32;
  karg_u32* p = (karg_u32*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t v[(NBYTES + 63) / 64];
#pragma unroll
  for (int i = 0; i < (NBYTES + 63) / 64; ++i) v[i] = p[16 * i];
#pragma unroll
  for (int i = 0; i < (NBYTES + 63) / 64; ++i) asm volatile("" ::"s"(v[i]));
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __builtin_bit_cast(float, bits16 << 16); }
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
// Two fp32 -> packed bf16x2 with round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Lane exchange with partner lane ^ HL inside a wave64, on the VALU (no LDS pipe):
//   1, 2  DPP quad_perm [1,0,3,2] / [2,3,0,1];
//   4     DPP row_half_mirror (i ^ 7) then quad_perm [3,2,1,0] (i ^ 3);
//   8     DPP row_ror:8 within the 16-lane row
//         (every lane's source lies in its row, so these moves need no fallback value);
//   16/32 v_permlane16_swap / v_permlane32_swap of the value with itself: the partner lands in the
//         first result on lanes with that lane bit set and in the second on the others.
// LDS_PIPE = true moves 4/8/16 to ds_swizzle (xor mode) and 32 to ds_bpermute instead: longer
// latency, but off the VALU, which pays in VALU-bound streaming kernels.
template <int HL, bool LDS_PIPE = false>
__device__ __forceinline__ float xor_lane(float v) {
  int i = __builtin_bit_cast(int, v);
  if constexpr (LDS_PIPE && (HL == 4 || HL == 8 || HL == 16)) {
    i = __builtin_amdgcn_ds_swizzle(i, (HL << 10) | 0x1F);
  } else if constexpr (LDS_PIPE && HL == 32) {
    i = __builtin_amdgcn_ds_bpermute(static_cast<int>(((threadIdx.x & 63) ^ 32) << 2), i);
  } else if constexpr (HL == 1) {
    i = __builtin_amdgcn_mov_dpp(i, 0xB1, 0xF, 0xF, false);
  } else if constexpr (HL == 2) {
    i = __builtin_amdgcn_mov_dpp(i, 0x4E, 0xF, 0xF, false);
  } else if constexpr (HL == 4) {
    i = __builtin_amdgcn_mov_dpp(i, 0x141, 0xF, 0xF, false);
    i = __builtin_amdgcn_mov_dpp(i, 0x1B, 0xF, 0xF, false);
  } else if constexpr (HL == 8) {
    i = __builtin_amdgcn_mov_dpp(i, 0x128, 0xF, 0xF, false);
  } else if constexpr (HL == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(i), static_cast<uint32_t>(i), false, false);
    i = static_cast<int>((threadIdx.x & 16) ? r[0] : r[1]);
  } else {
    static_assert(HL == 32, "xor_lane: HL must be a power of two below 64");
    const auto r = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(i), static_cast<uint32_t>(i), false, false);
    i = static_cast<int>((threadIdx.x & 32) ? r[0] : r[1]);
  }
  return __builtin_bit_cast(float, i);
}

// p[i] when p is set, else dflt.  The load is unconditional (from `fallback`, any readable word,
// when p is null), so it joins the caller's other loads in one memory round: a load under a branch
// is given its own wait by the compiler.
__device__ __forceinline__ int32_t load_or(const int32_t* p, int64_t i, const void* fallback, int32_t dflt) {
  const int32_t v = *(p ? p + i : static_cast<const int32_t*>(fallback));
  return p ? v : dflt;
}

__device__ __forceinline__ float xor_lane_rt(float v, int hl) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_ds_bpermute(static_cast<int>(((threadIdx.x & 63) ^ hl) << 2), __builtin_bit_cast(int, v)));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += xor_lane<1>(v);
  v += xor_lane<2>(v);
  v += xor_lane<4>(v);
  v += xor_lane<8>(v);
  v += xor_lane<16>(v);
  v += xor_lane<32>(v);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, xor_lane<1>(v));
  v = fmaxf(v, xor_lane<2>(v));
  v = fmaxf(v, xor_lane<4>(v));
  v = fmaxf(v, xor_lane<8>(v));
  v = fmaxf(v, xor_lane<16>(v));
  v = fmaxf(v, xor_lane<32>(v));
  return v;
}

// fp32 score -> uint32 whose unsigned order equals the float order (-inf smallest).
// (negative: every bit flipped; otherwise the sign bit set: u ^ (sign mask | 0x80000000))
__device__ __forceinline__ uint32_t order_key(float s) {
  const uint32_t u = __builtin_bit_cast(uint32_t, s);
  return u ^ (static_cast<uint32_t>(static_cast<int32_t>(u) >> 31) | 0x80000000u);
}
__device__ __forceinline__ float order_key_inv(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __builtin_bit_cast(float, u);
}

}  // namespace aekv
