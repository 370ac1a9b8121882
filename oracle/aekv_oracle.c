/*
 * aekv_oracle.c — CPU restatement of the reference's compressed-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: it is loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and by nothing else.  The product
 * (deepseek-v4-codebase_amd/aetherkv + libaetherkv.so) never links, imports or calls it.
 *
 * Built by oracle/Makefile with gcc -O2 -ffp-contract=off (no fast-math, no FMA contraction), so
 * every fp32 operation below rounds exactly like the corresponding torch CPU eager kernel.
 * Functions that mirror fp32 torch arithmetic bit-for-bit say so; reductions whose torch order is
 * unspecified (einsum, sum over heads) are evaluated in double and documented as "exact-math"
 * references: the tests compare the GPU against them with an error bound.
 *
 * Reference paths are relative to the reference repository root.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define AEKVO_F32 0
#define AEKVO_F16 1
#define AEKVO_BF16 2

/* ------------------------------------------------------------------------------------------ */
/* scalar conversions                                                                          */
/* ------------------------------------------------------------------------------------------ */
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float aekvo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* c10::BFloat16 round-to-nearest-even (NaN -> 0x7FC0). */
uint16_t aekvo_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float aekvo_f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) {
    if (m == 0) return u2f(s);
    float v = (float)m * 0x1p-24f; /* subnormal: m * 2^-24 (exact) */
    return s ? -v : v;
  }
  if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
  return u2f(s | ((e + 112u) << 23) | (m << 13));
}

/* IEEE binary16 round-to-nearest-even. */
uint16_t aekvo_f32_to_f16(float f) {
  uint32_t u = f2u(f), s = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(s | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u); /* rounds to >= 65520 -> inf */
  if (a < 0x38800000u) {                                 /* result subnormal or zero   */
    float v = u2f(a) * 0x1p24f;                          /* exact scaling, < 1024      */
    float r = nearbyintf(v);                             /* RNE at 2^-24 granularity   */
    return (uint16_t)(s | (uint32_t)r);
  }
  uint32_t mant = a & 0x7fffffu, exp = (a >> 23) - 112u;
  uint32_t half = (exp << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u;
  return (uint16_t)(s | half);
}

static inline float load_elem(const void* p, int dtype, int64_t i) {
  if (dtype == AEKVO_F32) return ((const float*)p)[i];
  if (dtype == AEKVO_BF16) return aekvo_bf16_to_f32(((const uint16_t*)p)[i]);
  return aekvo_f16_to_f32(((const uint16_t*)p)[i]);
}

static inline void store_elem(void* p, int dtype, int64_t i, float v) {
  if (dtype == AEKVO_F32) ((float*)p)[i] = v;
  else if (dtype == AEKVO_BF16) ((uint16_t*)p)[i] = aekvo_f32_to_bf16(v);
  else ((uint16_t*)p)[i] = aekvo_f32_to_f16(v);
}

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}

/* ------------------------------------------------------------------------------------------ */
/* Rademacher diagonal — aether_2b/turbo_quant.py:111-121                                        */
/* torch.Generator().manual_seed(seed*10007 + d); torch.rand(d): MT19937 (Matsumoto & Nishimura  */
/* 1998) seeded with the low 32 bits, float draw = (u32 & 0xFFFFFF) * 2^-24; diag = r>0.5?1:-1.  */
/* ------------------------------------------------------------------------------------------ */
typedef struct { uint32_t mt[624]; int idx; } mt19937_t;

static void mt_seed(mt19937_t* g, uint32_t s) {
  g->mt[0] = s;
  for (int i = 1; i < 624; ++i) g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + (uint32_t)i;
  g->idx = 624;
}

static uint32_t mt_next(mt19937_t* g) {
  if (g->idx >= 624) {
    for (int i = 0; i < 624; ++i) {
      uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
      g->mt[i] = g->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
    }
    g->idx = 0;
  }
  uint32_t y = g->mt[g->idx++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

void aekvo_diag(int64_t seed, int d, float* out) {
  mt19937_t g;
  mt_seed(&g, (uint32_t)((uint64_t)(seed * 10007 + d) & 0xffffffffu));
  for (int i = 0; i < d; ++i) {
    float r = (float)(mt_next(&g) & 0xffffffu) * 0x1p-24f;
    out[i] = r > 0.5f ? 1.0f : -1.0f;
  }
}

/* ------------------------------------------------------------------------------------------ */
/* Walsh-Hadamard transform — aether_2b/turbo_quant.py:49-76                                    */
/* Stage h = 1,2,..,d/2: within each 2h-block, out = cat([a+b, a-b]) with a = first h, b = next  */
/* h (fp32 add/sub); then multiply by fp32(d**-0.5) (python float cast to fp32 by torch).       */
/* ------------------------------------------------------------------------------------------ */
float aekvo_wht_scale(int d) { return (float)pow((double)d, -0.5); }

static void wht_inplace(float* v, float* tmp, int d) {
  for (int h = 1; h < d; h <<= 1) {
    for (int blk = 0; blk < d; blk += 2 * h) {
      for (int i = 0; i < h; ++i) {
        float a = v[blk + i], b = v[blk + h + i];
        tmp[blk + i] = a + b;
        tmp[blk + h + i] = a - b;
      }
    }
    memcpy(v, tmp, sizeof(float) * (size_t)d);
  }
  const float c = aekvo_wht_scale(d);
  for (int i = 0; i < d; ++i) v[i] = v[i] * c;
}

int aekvo_is_pow2(int d) { return d > 0 && (d & (d - 1)) == 0; }

int aekvo_wht(const void* x, int x_dtype, int64_t n, int d, float* out, int threads) {
  if (!aekvo_is_pow2(d)) return 1;
  set_threads(threads);
#pragma omp parallel
  {
    float* tmp = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
      float* v = out + r * d;
      for (int i = 0; i < d; ++i) v[i] = load_elem(x, x_dtype, r * d + i);
      wht_inplace(v, tmp, d);
    }
    free(tmp);
  }
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* PolarQuant.encode — aether_2b/turbo_quant.py:127-166                                         */
/*   rotated = _wht(x.float() * diag)                                                            */
/*   max_abs = rotated.abs().amax(-1).clamp_(min=1e-8)        (1e-8 cast to fp32)               */
/*   scale   = max_abs / Q                                      Q = 127.0 or 7.0                 */
/*   q       = (rotated / max_abs * Q).round_().clamp_(-Q, Q)   (round = half-to-even)          */
/*   8-bit: int8(q); 4-bit: byte i = (q[2i] & 15) | ((q[2i+1] & 15) << 4)                        */
/* ------------------------------------------------------------------------------------------ */
int aekvo_encode(const void* x, int x_dtype, int64_t n, int d, int bits, const float* diag,
                 uint8_t* codes, float* scale, int threads) {
  if (!aekvo_is_pow2(d) || (bits != 4 && bits != 8) || (bits == 4 && d < 2)) return 1;
  const float Q = bits == 8 ? 127.0f : 7.0f;
  const float eps = (float)1e-8;
  set_threads(threads);
#pragma omp parallel
  {
    float* v = (float*)malloc(sizeof(float) * (size_t)d);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
      for (int i = 0; i < d; ++i) v[i] = load_elem(x, x_dtype, r * d + i) * diag[i];
      wht_inplace(v, tmp, d);
      float m = 0.0f;
      for (int i = 0; i < d; ++i) { float a = fabsf(v[i]); if (a > m) m = a; }
      if (m < eps) m = eps;
      scale[r] = m / Q;
      if (bits == 8) {
        int8_t* o = (int8_t*)codes + r * d;
        for (int i = 0; i < d; ++i) {
          float t = v[i] / m;
          t = t * Q;
          t = nearbyintf(t);
          if (t > Q) t = Q;
          if (t < -Q) t = -Q;
          o[i] = (int8_t)(int)t;
        }
      } else {
        uint8_t* o = codes + r * (d / 2);
        for (int i = 0; i < d / 2; ++i) {
          int qv[2];
          for (int k = 0; k < 2; ++k) {
            float t = v[2 * i + k] / m;
            t = t * Q;
            t = nearbyintf(t);
            if (t > Q) t = Q;
            if (t < -Q) t = -Q;
            qv[k] = (int)t;
          }
          o[i] = (uint8_t)((qv[0] & 0x0f) | ((qv[1] & 0x0f) << 4));
        }
      }
    }
    free(v);
    free(tmp);
  }
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* PolarQuant.decode — aether_2b/turbo_quant.py:168-211                                         */
/*   8-bit: rotated = float(data) * scale                                                        */
/*   4-bit: even = b & 15, odd = (b >> 4) & 15, v >= 8 -> v - 16, interleave, * scale            */
/*   x = _wht(rotated) * diag  -> out_dtype (RNE)                                                */
/* ------------------------------------------------------------------------------------------ */
static inline void decode_row_f32(const uint8_t* codes, float s, int d, int bits, const float* diag,
                                  float* v, float* tmp, int64_t r) {
  if (bits == 8) {
    const int8_t* c = (const int8_t*)codes + r * d;
    for (int i = 0; i < d; ++i) v[i] = (float)c[i] * s;
  } else {
    const uint8_t* c = codes + r * (d / 2);
    for (int i = 0; i < d / 2; ++i) {
      int e = c[i] & 0x0f, o = (c[i] >> 4) & 0x0f;
      if (e >= 8) e -= 16;
      if (o >= 8) o -= 16;
      v[2 * i] = (float)e * s;
      v[2 * i + 1] = (float)o * s;
    }
  }
  wht_inplace(v, tmp, d);
  for (int i = 0; i < d; ++i) v[i] = v[i] * diag[i];
}

int aekvo_decode(const uint8_t* codes, const float* scale, int64_t n, int d, int bits,
                 const float* diag, void* out, int out_dtype, int threads) {
  if (!aekvo_is_pow2(d) || (bits != 4 && bits != 8) || (bits == 4 && d < 2)) return 1;
  set_threads(threads);
#pragma omp parallel
  {
    float* v = (float*)malloc(sizeof(float) * (size_t)d);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
      decode_row_f32(codes, scale[r], d, bits, diag, v, tmp, r);
      for (int i = 0; i < d; ++i) store_elem(out, out_dtype, r * d + i, v[i]);
    }
    free(v);
    free(tmp);
  }
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* CSA indexer scores (exact-math, double) — three reference rules:                            */
/*   mode 0 softplus : aether_2b/modeling.py:609-611 (and :521-523)                             */
/*                     score = sum_h softplus(w_h) * relu(q_h . k)                               */
/*   mode 1 raw      : aether_2b/serving.py:618-619  score = sum_h w_h * relu(q_h . k)           */
/*   mode 2 relu_w   : aether_kernels/csrc/csa_indexer_cuda.cu:44-55                           */
/*                     score = sum_{h: w_h > 0} w_h * (q_h . k)                                  */
/* softplus = torch.nn.functional.softplus(beta=1, threshold=20): x > 20 ? x : log1p(exp(x)).   */
/* keys: fp32 [B,S,IC]; scores double [B,S]; j >= valid[b] -> -inf (modeling.py:612-614).       */
/* ------------------------------------------------------------------------------------------ */
double aekvo_softplus(double x) { return x > 20.0 ? x : log1p(exp(x)); }

int aekvo_index_scores(const float* q, const float* w, const float* keys, const int32_t* valid,
                       int64_t B, int64_t S, int IH, int IC, int mode, double* scores, int threads) {
  set_threads(threads);
  for (int64_t b = 0; b < B; ++b) {
    double wa[64];
    if (IH > 64) return 1;
    for (int h = 0; h < IH; ++h) {
      double wv = w[b * IH + h];
      wa[h] = mode == 0 ? aekvo_softplus(wv) : wv;
    }
    const int64_t nv = valid ? valid[b] : S;
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < S; ++j) {
      if (j >= nv) { scores[b * S + j] = -INFINITY; continue; }
      const float* k = keys + (b * S + j) * IC;
      double acc = 0.0;
      for (int h = 0; h < IH; ++h) {
        const float* qh = q + (b * IH + h) * IC;
        double dot = 0.0;
        for (int c = 0; c < IC; ++c) dot += (double)qh[c] * (double)k[c];
        if (mode == 2) {
          if (wa[h] > 0.0) acc += wa[h] * dot;
        } else {
          acc += wa[h] * (dot > 0.0 ? dot : 0.0);
        }
      }
      scores[b * S + j] = acc;
    }
  }
  return 0;
}

/* Top-k under the total order (score desc, index asc); rows with fewer than k finite-or-not
 * candidates (j >= valid) are padded with -1.  Output sorted in that order. */
typedef struct { double s; int64_t i; } aekvo_pair;
static int pair_cmp(const void* a, const void* b) {
  const aekvo_pair* x = (const aekvo_pair*)a;
  const aekvo_pair* y = (const aekvo_pair*)b;
  if (x->s > y->s) return -1;
  if (x->s < y->s) return 1;
  return x->i < y->i ? -1 : (x->i > y->i ? 1 : 0);
}

int aekvo_topk(const double* scores, const int32_t* valid, int64_t B, int64_t S, int k,
               int64_t* out_idx, double* out_score) {
  aekvo_pair* p = (aekvo_pair*)malloc(sizeof(aekvo_pair) * (size_t)(S > 0 ? S : 1));
  for (int64_t b = 0; b < B; ++b) {
    const int64_t nv = valid ? (valid[b] < S ? valid[b] : S) : S;
    for (int64_t j = 0; j < nv; ++j) { p[j].s = scores[b * S + j]; p[j].i = j; }
    qsort(p, (size_t)nv, sizeof(aekvo_pair), pair_cmp);
    for (int t = 0; t < k; ++t) {
      out_idx[b * k + t] = t < nv ? p[t].i : -1;
      if (out_score) out_score[b * k + t] = t < nv ? p[t].s : -INFINITY;
    }
  }
  free(p);
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Sparse sink attention (exact-math, double accumulation).                                     */
/* aether_pipeline/serving.py:99-143 (PytorchAttentionBackend.sparse_attention), with the CUDA   */
/* kernel's out-of-range rule (aether_kernels/csrc/sparse_sink_attention_cuda.cu:79,105: index   */
/* outside [0,S) contributes nothing).                                                          */
/*   l_j = scale * q.K[idx_j];  M = max(max_j l_j, sink_h)                                       */
/*   out = sum_j e^{l_j-M} V[idx_j] / (sum_j e^{l_j-M} + e^{sink_h-M})   (duplicates counted)    */
/* A target with no index in range gets 0 whatever its sink (the kernel's weighted sum visits    */
/* only in-range indices, :102-113, so with the sink at -inf its NaN normaliser is never used).  */
/* q [B,T,H,D], kv [B,S,2,D], idx [B,T,K] (int64), sink [sink_numel] fp32; out fp32.            */
/* ------------------------------------------------------------------------------------------ */
int aekvo_sink_attention(const float* q, const float* kv, const int64_t* idx, const float* sink,
                         int64_t sink_numel, int64_t B, int64_t T, int64_t H, int64_t D, int64_t S,
                         int64_t K, double scale, float* out, int threads) {
  set_threads(threads);
#pragma omp parallel
  {
    double* l = (double*)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(static) collapse(2)
    for (int64_t bt = 0; bt < B * T; ++bt) {
      for (int64_t h = 0; h < H; ++h) {
        const int64_t b = bt / T;
        const float* qp = q + (bt * H + h) * D;
        const int64_t* ip = idx + bt * K;
        const double sk = sink_numel == 1 ? sink[0] : sink[h];
        double M = sk;
        for (int64_t j = 0; j < K; ++j) {
          const int64_t s = ip[j];
          if (s < 0 || s >= S) { l[j] = -INFINITY; continue; }
          const float* kp = kv + ((b * S + s) * 2 + 0) * D;
          double dot = 0.0;
          for (int64_t d = 0; d < D; ++d) dot += (double)qp[d] * (double)kp[d];
          l[j] = dot * scale;
          if (l[j] > M) M = l[j];
        }
        double den = exp(sk - M);
        int64_t n_in = 0;
        for (int64_t d = 0; d < D; ++d) acc[d] = 0.0;
        for (int64_t j = 0; j < K; ++j) {
          const int64_t s = ip[j];
          if (s < 0 || s >= S) continue;
          const double e = exp(l[j] - M);
          den += e;
          ++n_in;
          const float* vp = kv + ((b * S + s) * 2 + 1) * D;
          for (int64_t d = 0; d < D; ++d) acc[d] += e * (double)vp[d];
        }
        float* op = out + (bt * H + h) * D;
        for (int64_t d = 0; d < D; ++d) op[d] = n_in ? (float)(acc[d] / den) : 0.0f;
      }
    }
    free(l);
    free(acc);
  }
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Quantised decode-step attention (exact-math on the reference's bf16 operands).             */
/* aether_2b/serving.py:597-625 (CSA) and :507-522 (HCA): the resident cache is dequantised to  */
/* the model dtype (bf16, _read_compressed :346-376), the selected rows are gathered (:622-623,  */
/* full range for HCA), the bf16 window is appended (:624), K = V = source (:52-53), and         */
/* PytorchAttentionBackend attends with the sink.  sel == NULL: all S blocks.  sel entries      */
/* outside [0,S) are skipped.  q [B,H,D] fp32 (bf16 values), window [B,W,D] fp32 (bf16 values), */
/* codes/scale as PolarQuant; out [B,H,D] fp32.                                                 */
/* ------------------------------------------------------------------------------------------ */
int aekvo_quant_attention(const float* q, const uint8_t* codes, const float* scale,
                          const int64_t* sel, const float* window, const float* sink,
                          const float* diag, int64_t B, int64_t H, int64_t D, int64_t S, int64_t K,
                          int64_t W, int bits, double sm_scale, float* out, int threads) {
  set_threads(threads);
  const int64_t nsel = sel ? K : S;
  const int64_t row_bytes = bits == 8 ? D : D / 2;
#pragma omp parallel
  {
    float* src = (float*)malloc(sizeof(float) * (size_t)((nsel + W) * D + 1));
    float* tmp = (float*)malloc(sizeof(float) * (size_t)D);
    double* l = (double*)malloc(sizeof(double) * (size_t)(nsel + W + 1));
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
    char* ok = (char*)malloc((size_t)(nsel + W + 1));
#pragma omp for schedule(static)
    for (int64_t b = 0; b < B; ++b) {
      for (int64_t j = 0; j < nsel; ++j) {
        const int64_t s = sel ? sel[b * K + j] : j;
        ok[j] = (s >= 0 && s < S);
        if (!ok[j]) continue;
        float* v = src + j * D;
        decode_row_f32(codes + (b * S + s) * row_bytes, scale[b * S + s], (int)D, bits, diag, v, tmp, 0);
        for (int64_t d = 0; d < D; ++d) v[d] = aekvo_bf16_to_f32(aekvo_f32_to_bf16(v[d]));
      }
      for (int64_t w = 0; w < W; ++w) {
        ok[nsel + w] = 1;
        memcpy(src + (nsel + w) * D, window + (b * W + w) * D, sizeof(float) * (size_t)D);
      }
      const int64_t n = nsel + W;
      for (int64_t h = 0; h < H; ++h) {
        const float* qp = q + (b * H + h) * D;
        const double sk = sink[h];
        double M = sk;
        for (int64_t j = 0; j < n; ++j) {
          if (!ok[j]) continue;
          double dot = 0.0;
          for (int64_t d = 0; d < D; ++d) dot += (double)qp[d] * (double)src[j * D + d];
          l[j] = dot * sm_scale;
          if (l[j] > M) M = l[j];
        }
        double den = exp(sk - M);
        int64_t n_in = 0;
        for (int64_t d = 0; d < D; ++d) acc[d] = 0.0;
        for (int64_t j = 0; j < n; ++j) {
          if (!ok[j]) continue;
          const double e = exp(l[j] - M);
          den += e;
          ++n_in;
          for (int64_t d = 0; d < D; ++d) acc[d] += e * (double)src[j * D + d];
        }
        /* no source: 0, as the engine's empty-source step (aether_2b/serving.py:451-452) */
        for (int64_t d = 0; d < D; ++d) out[(b * H + h) * D + d] = n_in ? (float)(acc[d] / den) : 0.0f;
      }
    }
    free(src);
    free(tmp);
    free(l);
    free(acc);
    free(ok);
  }
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* HCA window compression — aether_2b/serving.py:495-497 (_hca_emit) and the hca_compress API   */
/* (aether_kernels/sparse_attention.py:70-83): out[b,d] = sum_m softmax_m(z[b,:,d]) c[b,m,d].   */
/* Exact-math (double).                                                                          */
/* ------------------------------------------------------------------------------------------ */
int aekvo_hca_compress(const float* c, const float* z, int64_t B, int64_t M, int64_t D, float* out) {
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t d = 0; d < D; ++d) {
      double mx = -INFINITY;
      for (int64_t m = 0; m < M; ++m) { double v = z[(b * M + m) * D + d]; if (v > mx) mx = v; }
      double den = 0.0, acc = 0.0;
      for (int64_t m = 0; m < M; ++m) {
        const double e = exp((double)z[(b * M + m) * D + d] - mx);
        den += e;
        acc += e * (double)c[(b * M + m) * D + d];
      }
      out[b * D + d] = (float)(acc / den);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Block emission — aether_2b/serving.py:495-505 (_hca_emit) and :557-576 (_emit_csa_block,     */
/* main and index parts), modeling.py:122-155 (apply_rope), :32-41 (RMSNorm).  bf16 tensors in  */
/* and out, at torch CPU's rounding points (tests/test_oracle.py pins this against torch):       */
/*   zz  = bf16(z + bias)                         (bias optional: the CSA per-slot biases)       */
/*   w_m = bf16(exp(zz_m - max) * (1 / sum_m exp(zz_m - max)))   fp32, sums in m order          */
/*   x   = bf16(sum_m float(bf16(w_m * c_m)))      fp32 sum in m order                          */
/*   RoPE on the last rope_dim dims (pairs (2i, 2i+1) of that part), cos/sin =                   */
/*     bf16(cos/sin(fp32(pos) * inv_freq[i])): even bf16(bf16(a cos) + bf16(-b sin)),            */
/*     odd bf16(bf16(b cos) + bf16(a sin))                                                        */
/*   RMSNorm: r = 1 / sqrt(mean(x^2) + eps) (fp32, sum in d order); y = bf16((x * r) * w)        */
/* ------------------------------------------------------------------------------------------ */
static inline float bf(float v) { return aekvo_bf16_to_f32(aekvo_f32_to_bf16(v)); }

/* apply_rope (modeling.py:122-155) at fp32 position p on the last rope_dim dims, then RMSNorm
 * (modeling.py:32-41) when norm_w is given, in place on a bf16-valued vector x[D]. */
static void rope_rmsnorm_vec(float* x, int64_t D, int rope_dim, float p, const float* inv_freq,
                             const uint16_t* norm_w, float eps) {
  if (rope_dim > 0) {
    const int64_t r0 = D - rope_dim;
    for (int i = 0; i < rope_dim / 2; ++i) {
      const float ang = p * inv_freq[i];
      const float cs = bf(cosf(ang)), sn = bf(sinf(ang));
      const float a = x[r0 + 2 * i], bb = x[r0 + 2 * i + 1];
      x[r0 + 2 * i] = bf(bf(a * cs) + bf(-bb * sn));
      x[r0 + 2 * i + 1] = bf(bf(bb * cs) + bf(a * sn));
    }
  }
  if (norm_w) {
    float ss = 0.0f;
    for (int64_t d = 0; d < D; ++d) ss += x[d] * x[d];
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
    for (int64_t d = 0; d < D; ++d) x[d] = bf((x[d] * r) * aekvo_bf16_to_f32(norm_w[d]));
  }
}

/* Query / window-entry preparation and inverse RoPE of the attention output (aether_2b/serving.py:
 * 437-448, 469-472): x [rows * heads, D] bf16, vector (row n, head h) at fp32 position
 * sign * pos[n]; rope then (optional) RMSNorm as rope_rmsnorm_vec. */
int aekvo_rope_rmsnorm(const uint16_t* x, int64_t rows, int64_t heads, int64_t D, const int64_t* pos, int sign,
                       const float* inv_freq, int rope_dim, const uint16_t* norm_w, float eps, uint16_t* out) {
  if (rows < 0 || heads < 1 || D < 2 || rope_dim < 0 || rope_dim > D || (rope_dim & 1)) return 1;
  if (sign != 1 && sign != -1) return 1;
  float* v = (float*)malloc(sizeof(float) * (size_t)D);
  if (!v) return 2;
  for (int64_t n = 0; n < rows; ++n)
    for (int64_t h = 0; h < heads; ++h) {
      const uint16_t* xr = x + (n * heads + h) * D;
      for (int64_t d = 0; d < D; ++d) v[d] = aekvo_bf16_to_f32(xr[d]);
      rope_rmsnorm_vec(v, D, rope_dim, rope_dim > 0 ? (float)((int64_t)sign * pos[n]) : 0.0f, inv_freq, norm_w, eps);
      for (int64_t d = 0; d < D; ++d) out[(n * heads + h) * D + d] = aekvo_f32_to_bf16(v[d]);
    }
  free(v);
  return 0;
}

int aekvo_emit_block(const uint16_t* c, const uint16_t* z, const uint16_t* bias, int64_t B, int64_t L, int64_t D,
                     int rope_dim, const int64_t* pos, const float* inv_freq, const uint16_t* norm_w, float eps,
                     uint16_t* out) {
  if (B < 0 || L < 1 || D < 1 || rope_dim < 0 || rope_dim > D || (rope_dim & 1)) return 1;
  float* x = (float*)malloc(sizeof(float) * (size_t)D);
  float* e = (float*)malloc(sizeof(float) * (size_t)L);
  if (!x || !e) { free(x); free(e); return 2; }
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t d = 0; d < D; ++d) {
      float mx = -INFINITY;
      for (int64_t m = 0; m < L; ++m) {
        float zz = aekvo_bf16_to_f32(z[(b * L + m) * D + d]);
        if (bias) zz = bf(zz + aekvo_bf16_to_f32(bias[m * D + d]));
        e[m] = zz;
        if (zz > mx) mx = zz;
      }
      float sum = 0.0f;
      for (int64_t m = 0; m < L; ++m) { e[m] = expf(e[m] - mx); sum += e[m]; }
      const float inv = 1.0f / sum;
      float acc = 0.0f;
      for (int64_t m = 0; m < L; ++m) {
        const float w = bf(e[m] * inv);
        acc += bf(w * aekvo_bf16_to_f32(c[(b * L + m) * D + d]));
      }
      x[d] = bf(acc);
    }
    rope_rmsnorm_vec(x, D, rope_dim, rope_dim > 0 ? (float)pos[b] : 0.0f, inv_freq, norm_w, eps);
    for (int64_t d = 0; d < D; ++d) out[b * D + d] = aekvo_f32_to_bf16(x[d]);
  }
  free(x);
  free(e);
  return 0;
}
