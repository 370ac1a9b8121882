/*
 * aetherkv.h — C ABI of libaetherkv.so, the MI355X (gfx950) compressed-KV hot path.
 *
 * Every entry point:
 *   - is extern "C", takes plain device pointers, int64 sizes and a hipStream_t passed as void*;
 *   - validates every argument on the host BEFORE any launch (so argument errors are testable
 *     without a GPU) and returns an aekv_status; the message of the last failure on the calling
 *     thread is returned by aekv_last_error();
 *   - never allocates device memory: scratch space is passed in (`ws`, `ws_bytes`) and its size
 *     is returned by the matching *_workspace_size() query;
 *   - enqueues its kernels on `stream` and returns without synchronising.
 *
 * Reference interfaces replaced (paths relative to the reference repository root):
 *   aekv_wht                         aether_2b/turbo_quant.py:49-76             _wht(x)
 *   aekv_tq_diag                     aether_2b/turbo_quant.py:111-121           PolarQuant._diag(d, device)
 *   aekv_tq_encode                   aether_2b/turbo_quant.py:127-166           PolarQuant.encode(x)
 *   aekv_tq_decode                   aether_2b/turbo_quant.py:168-211           PolarQuant.decode(data, scale, out_dtype)
 *   aekv_csa_indexer_topk            aether_kernels/sparse_attention.py:45-67   csa_indexer_topk(...)
 *                                    (binding aether_kernels/csrc/bindings.cpp:88-101)
 *   aekv_csa_indexer_topk_quant      aether_2b/serving.py:606-621 (indexer over the quantised index cache)
 *   aekv_sparse_sink_attention       aether_kernels/sparse_attention.py:8-16    sparse_sink_attention(...)
 *                                    (binding aether_kernels/csrc/bindings.cpp:21-46)
 *   aekv_quant_sink_attention        aether_2b/serving.py:507-525 (HCA) and :597-625 (CSA): dequantise,
 *                                    gather, concat window, aether_pipeline/serving.py:99-130 attention
 *   aekv_hca_compress                aether_kernels/sparse_attention.py:70-83   hca_compress(...)
 *   aekv_emit_block                  aether_2b/serving.py:495-505 (_hca_emit) and :557-576
 *                                    (_emit_csa_block): pool + RoPE + kv_norm + _quant_append
 *   aekv_tiled_prefill_attention     aether_kernels/sparse_attention.py:19-42   tiled_prefill_attention(...)
 *   aekv_csa_decode_quant            aether_2b/serving.py:597-625 (the CSA decode step: indexer, topk, gather,
 *                                    window concat and sink attention)
 */
#ifndef AETHERKV_H_
#define AETHERKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------------------- */
typedef enum {
  AEKV_OK = 0,
  AEKV_ERR_VALUE = 1,       /* bad value (bits, non-power-of-two dim, k, ...)  -> ValueError   */
  AEKV_ERR_SHAPE = 2,       /* inconsistent shapes / ranks                     -> RuntimeError */
  AEKV_ERR_DTYPE = 3,       /* unsupported dtype                               -> RuntimeError */
  AEKV_ERR_ALIGN = 4,       /* pointer not aligned as documented               -> RuntimeError */
  AEKV_ERR_WORKSPACE = 5,   /* ws NULL or ws_bytes smaller than the query      -> RuntimeError */
  AEKV_ERR_HIP = 6,         /* a HIP launch/runtime call failed                -> RuntimeError */
  AEKV_ERR_UNSUPPORTED = 7  /* size outside what the kernels support           -> RuntimeError */
} aekv_status;

/* ---- element types ----------------------------------------------------------------------- */
typedef enum {
  AEKV_F32 = 0,
  AEKV_F16 = 1,
  AEKV_BF16 = 2,
  AEKV_I32 = 3,
  AEKV_I64 = 4
} aekv_dtype;

/* Indexer score rules.  The reference has three (file:line of each):
 *   AEKV_IDX_SOFTPLUS : sum_h softplus(w_h) * relu(q_h . k_j)   aether_2b/modeling.py:609-611, :521-523
 *   AEKV_IDX_RAW      : sum_h w_h * relu(q_h . k_j)             aether_2b/serving.py:618-619
 *   AEKV_IDX_RELU_W   : sum_h max(w_h, 0) * (q_h . k_j)         aether_kernels/csrc/csa_indexer_cuda.cu:44-55 */
typedef enum {
  AEKV_IDX_SOFTPLUS = 0,
  AEKV_IDX_RAW = 1,
  AEKV_IDX_RELU_W = 2
} aekv_index_mode;

/* ---- library ----------------------------------------------------------------------------- */
const char* aekv_version(void);
/* Message of the last non-OK status returned on the calling thread ("" if none). */
const char* aekv_last_error(void);
/* Largest supported values (compile-time limits of the kernels). */
int32_t aekv_max_head_dim(void);   /* power-of-two vector length limit for the codec (512)   */
int32_t aekv_max_topk(void);       /* largest k accepted by the indexer select (2048)         */
/* Kernel selection (no reference counterpart; a testing and A/B aid): 1 = use only the generic
 * kernels, 0 = also use the kernels specialised for the production shape (default, unless the
 * environment sets AETHERKV_CODEC=generic).  Both produce identical results.  Returns the
 * previous setting. */
int aekv_set_generic_kernels(int generic_only);
/* Workgroup shape of the HCA prefill flash kernel (no reference counterpart; a testing and A/B
 * aid): 0 = chosen per launch (default), 64 = four waves over 64 (target, head) rows, 96 = twelve
 * waves over 96 rows.  Both compute the same attention within the bf16 tolerance (they split
 * and merge each row's keys differently, so single outputs may differ in the last bit).  Returns
 * the previous setting (0, 64 or 96), or AEKV_ERR_VALUE (1) for any other value, which changes
 * nothing. */
int aekv_set_flash_rows(int rows);

/* ---- TurboQuant codec -------------------------------------------------------------------- */
/* Rademacher diagonal of PolarQuant(seed)._diag(d): MT19937 seeded with seed*10007+d, one
 * 32-bit draw per element, r = (draw & 0xFFFFFF) * 2^-24, diag = r > 0.5 ? +1 : -1.
 * Host memory out[d].  (turbo_quant.py:111-121; torch.rand's CPU generator is MT19937.) */
int aekv_tq_diag(int64_t seed, int32_t d, float* out_host);

/* Normalised Walsh-Hadamard transform of n_vec rows of length d (power of two, 1..512):
 * x (x_dtype f32/f16/bf16) -> out fp32, butterfly stages h = 1,2,..,d/2 in order, then * fp32(d^-0.5).
 * x must be aligned to min(d,8)*sizeof(x_dtype) bytes, out to min(d,8)*4. */
int aekv_wht(const void* x, int32_t x_dtype, int64_t n_vec, int32_t d, float* out, void* stream);

/* Encode: rot = WHT(x * diag); m = max(max|rot|, 1e-8); scale = m / Q; codes = clamp(rne(rot/m*Q))
 * with Q = 127 (bits 8: int8 codes [n_vec, d]) or Q = 7 (bits 4: uint8 [n_vec, d/2], element 2i in
 * the low nibble, 2i+1 in the high nibble, two's complement).  scale fp32 [n_vec].
 * diag: device fp32 [d] of +-1.  Bit-exact with turbo_quant.py:127-166. */
int aekv_tq_encode(const void* x, int32_t x_dtype, int64_t n_vec, int32_t d, int32_t bits,
                   const float* diag, void* codes, float* scale, void* stream);

/* Decode: rot = codes * scale; out = WHT(rot) * diag, rounded to out_dtype (f32/f16/bf16, RNE).
 * Bit-exact with turbo_quant.py:168-211. */
int aekv_tq_decode(const void* codes, const float* scale, int64_t n_vec, int32_t d, int32_t bits,
                   const float* diag, void* out, int32_t out_dtype, void* stream);

/* ---- CSA indexer + top-k ----------------------------------------------------------------- */
/* Scores score[b,j] = sum_h act(w[b,h]) * rho(q[b,h,:] . k[b,j,:]) (act/rho from `mode`) for
 * j < valid[b] (valid == NULL: all S), and returns the k best per row under the total order
 * (score descending, index ascending), sorted in that order, as int64 out_idx[B, k].  Rows with
 * valid[b] < k are padded with -1.  out_score[B, k] (fp32, nullable) receives the scores.
 *
 * aekv_csa_indexer_topk: fp32 keys index_kv[B, S, IC] (drop-in for csa_indexer_topk).
 * aekv_csa_indexer_topk_quant: keys are TurboQuant codes key_codes[B, S, IC or IC/2] with
 *   key_scale[B, S]; k_j = decode(codes_j, scale_j) in fp32.  The scan runs in the rotated domain:
 *   q.k_j = scale_j * (WHT(diag*q) . codes_j). */
size_t aekv_csa_indexer_workspace_size(int64_t B, int64_t S, int32_t k);
int aekv_csa_indexer_topk(const float* index_q, const float* index_kv, const float* index_weight,
                          const int32_t* valid, int64_t B, int64_t S, int32_t IH, int32_t IC,
                          int32_t k, int32_t mode, void* ws, size_t ws_bytes,
                          int64_t* out_idx, float* out_score, void* stream);
int aekv_csa_indexer_topk_quant(const float* index_q, const float* index_weight,
                                const void* key_codes, const float* key_scale, const float* diag,
                                const int32_t* valid, int64_t B, int64_t S, int32_t IH, int32_t IC,
                                int32_t bits, int32_t k, int32_t mode, void* ws, size_t ws_bytes,
                                int64_t* out_idx, float* out_score, void* stream);

/* Allocation-free variant of aekv_csa_indexer_topk_quant (same arguments and results, no ws/ws_bytes).
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Its scratch is a static
 * device array of AEKV_STATIC_SCRATCH_BYTES in the library, one per GPU, held until the process ends;
 * the first call on a device looks up its address (the current device must be the stream's).
 * Launches whose workspace, aekv_csa_indexer_workspace_size(B, S, k), exceeds it return
 * AEKV_ERR_UNSUPPORTED (cfg5, B = 64 x S = 65536, needs 17.8 MB).  It calls no allocating routine.
 * Every call on one GPU shares the array: calls that overlap on that GPU (other streams, other
 * threads) race and must be serialised by the caller. */
#define AEKV_STATIC_SCRATCH_BYTES ((size_t)32 << 20)
int aekv_csa_indexer_topk_quant_noalloc(const float* index_q, const float* index_weight,
                                        const void* key_codes, const float* key_scale, const float* diag,
                                        const int32_t* valid, int64_t B, int64_t S, int32_t IH, int32_t IC,
                                        int32_t bits, int32_t k, int32_t mode, int64_t* out_idx,
                                        float* out_score, void* stream);

/* Chunked-prefill variant: T targets per sequence (modeling.py:496-534, the per-target indexer of
 * _forward_tiled_prefill).  index_q [B,T,IH,IC], index_weight [B,T,IH], valid [B,T] (target t of
 * row b scores blocks j < valid[b,t] of key row b: its causally visible blocks), out_idx
 * [B,T,k], out_score [B,T,k]; keys as aekv_csa_indexer_topk_quant.  Workspace:
 * aekv_csa_indexer_workspace_size(B * T, S, k).  B * T <= 65535. */
int aekv_csa_prefill_indexer_topk_quant(const float* index_q, const float* index_weight,
                                        const void* key_codes, const float* key_scale, const float* diag,
                                        const int32_t* valid, int64_t B, int64_t T, int64_t S, int32_t IH,
                                        int32_t IC, int32_t bits, int32_t k, int32_t mode, void* ws,
                                        size_t ws_bytes, int64_t* out_idx, float* out_score, void* stream);

/* ---- attention ----------------------------------------------------------------------------- */
/* Drop-in sparse sink attention (sparse_sink_attention_cuda.cu semantics, oracle
 * aether_pipeline/serving.py:99-130):
 *   q [B,T,H,D], kv [B,S,2,D] (K = kv[:,:,0], V = kv[:,:,1]), topk [B,T,K] (idx_dtype I32/I64),
 *   sink: sink_numel == 1 (scalar) or H, same dtype as q.  Index outside [0,S) is skipped.
 *   out[b,t,h] = sum_j e^{l_j-M} V[idx_j] / (sum_j e^{l_j-M} + e^{sink_h-M}),
 *   l_j = scale * q.K[idx_j], M = max(max_j l_j, sink_h).  dtype F32/F16/BF16, D <= 512. */
int aekv_sparse_sink_attention(const void* q, const void* kv, const void* topk, int32_t idx_dtype,
                               const void* sink, int64_t sink_numel, int32_t dtype,
                               int64_t B, int64_t T, int64_t H, int64_t D, int64_t S, int64_t K,
                               float softmax_scale, void* out, void* stream);

/* The same, with a caller-owned workspace (the binding's own allocation in the reference,
 * bindings.cpp:21-46, happens in the caller here): bf16/fp16 calls at D = 128 whose launch would
 * leave most CUs idle split each target's sources over several workgroups and merge the pieces.
 * ws_bytes from aekv_sink_attention_workspace_size(dtype, B, T, H, D, S, K); ws = NULL runs unsplit
 * (the entry point above); a non-NULL ws must be 256-byte aligned and large enough. */
int aekv_sparse_sink_attention_ws(const void* q, const void* kv, const void* topk, int32_t idx_dtype,
                                  const void* sink, int64_t sink_numel, int32_t dtype,
                                  int64_t B, int64_t T, int64_t H, int64_t D, int64_t S, int64_t K,
                                  float softmax_scale, void* ws, size_t ws_bytes, void* out, void* stream);
/* Workspace bytes for the split of aekv_sparse_sink_attention_ws (K sources per target) or, with
 * K < 0, aekv_tiled_prefill_attention_ws (every target over all S sources); 0: no split. */
size_t aekv_sink_attention_workspace_size(int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t D, int64_t S,
                                          int64_t K);

/* Sink attention of one bf16 query token per row over TurboQuant-compressed shared K=V blocks plus
 * a bf16 sliding window (the serving engine's decode step, dequantise + gather + concat + attend
 * fused):
 *   q [B,H,D] bf16; codes [B,S,D or D/2] + scale [B,S]; sel [B,n_sel] int64 block indices
 *   (n_sel < 0: all S blocks in order, i.e. HCA, sel ignored; sel NULL with n_sel >= 0: the first
 *   min(n_sel, S) blocks of each row in order, S then being the row stride of codes and scale, e.g. a
 *   ring's storage holding n_sel valid blocks; entries outside [0,S) are skipped);
 *   window [B,W,D] bf16 (W may be 0); sink fp32 [H]; out [B,H,D] bf16.
 *   Sources = [dequant(blocks[sel]), window]; K = V = source (aether_2b/serving.py:52-53).
 * Gathered code rows are dequantised on load to the bf16 values the engine attends (its bf16
 * dequantised cache): exactly PolarQuant.decode's values on the generic path; on the matrix-core
 * path (D = 128, H <= 16) the transform runs as an exact int32 product and one fp32 scaling, at
 * most one bf16 ulp from PolarQuant.decode.  Logits and the value sum accumulate in fp32. */
size_t aekv_quant_attention_workspace_size(int64_t B, int64_t H, int64_t D, int64_t n_comp,
                                           int64_t W);
int aekv_quant_sink_attention(const void* q, const void* codes, const float* scale,
                              const int64_t* sel, const void* window, const float* sink,
                              const float* diag, int64_t B, int64_t H, int64_t D, int64_t S,
                              int64_t n_sel, int64_t W, int32_t bits, float softmax_scale,
                              void* ws, size_t ws_bytes, void* out, void* stream);

/* Chunked prefill through the quantised reader (modeling.py:293-337 HCA and :496-550 CSA
 * _forward_tiled_prefill, whose per-target tiled_prefill_attention calls, sparse_attention.py:19-42,
 * become one launch): target t of row b attends
 *   [dequant(blocks of its selection), window[b, win_start[b,t] : win_start[b,t] + win_len[b,t]]]
 * with K = V and the per-head sink.  Its blocks: sel[b,t,0 : visible[b,t]] (n_sel >= 0; entries
 * outside [0,S) skipped) or blocks 0 .. visible[b,t]-1 in order (n_sel < 0, HCA); visible NULL means
 * n_sel (or S).  win_start / win_len NULL mean 0 / the rest of the Wt entries; every count is
 * clamped to its buffer.  q [B,T,H,D] bf16, codes [B,S,D or D/2] + scale [B,S], window [B,Wt,D]
 * bf16, sink fp32 [H], out [B,T,H,D] bf16; a target with no sources gets zeros.  Dequantised values
 * as the matrix-core path of aekv_quant_sink_attention (D = 128, H <= 16 only; pointers 16-byte
 * aligned, out 8-byte).  Workspace: aekv_quant_prefill_workspace_size(B, T, H, n_comp, Wt) with
 * n_comp = n_sel (or S).  B * T <= 65535. */
size_t aekv_quant_prefill_workspace_size(int64_t B, int64_t T, int64_t H, int64_t n_comp, int64_t Wt);
int aekv_quant_prefill_attention(const void* q, const void* codes, const float* scale, const int64_t* sel,
                                 const int32_t* visible, const void* window, const int32_t* win_start,
                                 const int32_t* win_len, const float* sink, const float* diag, int64_t B,
                                 int64_t T, int64_t H, int64_t D, int64_t S, int64_t n_sel, int64_t Wt,
                                 int32_t bits, float softmax_scale, void* ws, size_t ws_bytes, void* out,
                                 void* stream);

/* One CSA decode step over TurboQuant-coded caches (aether_2b/serving.py:597-625: score every
 * visible block of the index cache, topk, gather the selected KV blocks, concat the window, attend
 * with the per-head sink): aekv_csa_indexer_topk_quant's selection (out_idx [B, k] int64, -1 padded,
 * out_score nullable) followed by aekv_quant_sink_attention over sel = out_idx, n_sel = k (out
 * [B, H, D] bf16), with the same results.  Where the matrix-core kernels apply (IH <= 16, IC 64 or
 * 128, k <= 512, D = 128, H <= 16, k + W <= 1024, 16-byte aligned q, codes, window and diag) the
 * selection and the attention run in one workgroup per row; otherwise the two entry points run in
 * turn.  Workspace: aekv_csa_decode_workspace_size(B, S, k, H, D, W). */
size_t aekv_csa_decode_workspace_size(int64_t B, int64_t S, int32_t k, int64_t H, int64_t D, int64_t W);
int aekv_csa_decode_quant(const float* index_q, const float* index_weight, const void* index_codes,
                          const float* index_scale, const float* index_diag, const int32_t* valid, int64_t B,
                          int64_t S, int32_t IH, int32_t IC, int32_t index_bits, int32_t k, int32_t mode,
                          const void* q, const void* kv_codes, const float* kv_scale, const void* window,
                          const float* sink, const float* kv_diag, int64_t H, int64_t D, int64_t W,
                          int32_t kv_bits, float softmax_scale, void* ws, size_t ws_bytes, int64_t* out_idx,
                          float* out_score, void* out, void* stream);

/* hca_compress drop-in: out[b,d] = sum_m softmax_m(z[b,:,d]) * c[b,m,d], c/z [B,M,D], dtype
 * F32/F16/BF16, out [B,D] same dtype (hca_compress_cuda.cu:18-68; serving.py:495-497). */
int aekv_hca_compress(const void* c, const void* z, int32_t dtype, int64_t B, int64_t M, int64_t D,
                      void* out, void* stream);

/* Block emission into a code ring: for each row b, pool the block's len token entries
 *   x = sum_m bf16(softmax_m(bf16(z + z_bias)) * c_m)      (c, z [B, len, d] bf16; z_bias [len, d]
 *                                                           bf16 or NULL; fp32 softmax and sums)
 * apply RoPE on the last rope_dim dims at positions[b] with frequencies inv_freq[rope_dim/2]
 * (rope_dim 0: none), RMSNorm with norm_weight[d] bf16 and eps (NULL: none), and write the
 * TurboQuant code of the result (bits 4/8, diag [d]) to out_codes + b*out_row_stride rows and
 * out_scale[b*out_row_stride] — i.e. out_codes/out_scale point at the block's slot of row 0 of a
 * [B, out_row_stride, ...] ring.  out_vec [B, d] bf16 (nullable) receives the vector before
 * encoding.  d = 64 or 128.  Rounding points as the reference's bf16 torch ops (softmax in fp32,
 * bf16 weights and products, fp32 sums, bf16 RoPE terms, fp32 RMSNorm); the encode is exactly
 * aekv_tq_encode's. */
int aekv_emit_block(const void* c, const void* z, const void* z_bias, int64_t B, int64_t len, int32_t d,
                    int32_t rope_dim, const int64_t* positions, const float* inv_freq,
                    const void* norm_weight, float eps, int32_t bits, const float* diag, void* out_codes,
                    float* out_scale, int64_t out_row_stride, void* out_vec, void* stream);

/* RoPE then RMSNorm of head vectors (the attention step's query and window-entry preparation,
 * aether_2b/serving.py:437-442 _query, :444-448 _window_entry; with pos_sign = -1 and no norm the
 * inverse RoPE of _post_attention, :469-472; apply_rope modeling.py:122-155, RMSNorm :32-41):
 * x [rows, heads, d] bf16; vector (n, h) is rotated on its last rope_dim dims at fp32 position
 * pos_sign * positions[n] with frequencies inv_freq[rope_dim/2] (rope_dim 0: none), then
 * normalised with norm_weight[d] bf16 and eps (NULL: none); out [rows, heads, d] bf16 (may alias
 * x).  Rounding points as the reference's bf16 torch ops (bf16 cos/sin and RoPE terms, fp32
 * RMSNorm).  d = 128 or 256. */
int aekv_rope_rmsnorm(const void* x, int64_t rows, int32_t heads, int32_t d, const int64_t* positions,
                      int32_t pos_sign, const float* inv_freq, int32_t rope_dim, const void* norm_weight,
                      float eps, void* out, void* stream);

/* tiled_prefill_attention drop-in: sink attention of every target over all S sources,
 * oracle aether_2b/modeling.py:158-178 (sink counted once in the normaliser). */
int aekv_tiled_prefill_attention(const void* q, const void* kv, const void* sink, int64_t sink_numel,
                                 int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t D, int64_t S,
                                 float softmax_scale, int32_t tile_size, void* out, void* stream);
/* The same with a caller-owned workspace (size: aekv_sink_attention_workspace_size(..., K = -1));
 * see aekv_sparse_sink_attention_ws. */
int aekv_tiled_prefill_attention_ws(const void* q, const void* kv, const void* sink, int64_t sink_numel,
                                    int32_t dtype, int64_t B, int64_t T, int64_t H, int64_t D, int64_t S,
                                    float softmax_scale, int32_t tile_size, void* ws, size_t ws_bytes, void* out,
                                    void* stream);

#ifdef __cplusplus
}
#endif
#endif /* AETHERKV_H_ */
