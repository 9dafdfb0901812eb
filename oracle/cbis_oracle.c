/*
 * cbis_oracle.c -- CPU restatement of the reference's per-step forward math.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP kernels, the
 * C-ABI libraries, the C++ runtime) links, loads or calls this file.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as
 * the checker / the timed CPU baseline.
 *
 * Every function restates the reference algorithm in fp64 and cites the
 * reference file:line it follows (paths relative to the reference root):
 *
 *   orc_gemm             kernels/linear.cu:15-34, docs/gemm_layout.md:16-41
 *                        (Y[M,N] = X[M,K] . W[N,K]^T + b), bias add
 *                        kernels/linear.cu:6-12, GELU kernels/elementwise.cu:59-66,
 *                        residual kernels/elementwise.cu:68-73
 *   orc_layernorm        kernels/elementwise.cu:21-57 (eps 1e-5, biased variance)
 *                        == python/model.py:26 nn.LayerNorm
 *   orc_embed            kernels/elementwise.cu:7-17, python/model.py:66-67
 *   orc_paged_attention  kernels/attention.cu:57-98 (kv_len = pos+1, scale
 *                        1/sqrt(hd), page addressing [page][slot][head][dim],
 *                        row_page_table lookup), python/model.py:35-46 (causal
 *                        softmax attention)
 *   orc_scatter_kv       kernels/attention.cu:7-19
 *   orc_forward_step     src/transformer.cpp:44-99 (op order; scatter before
 *                        attention of the same layer; lm_head without bias,
 *                        python/model.py:61), also in parts:
 *                        orc_step_embed / orc_step_layer / orc_step_head
 *   orc_argmax           src/bench_batching.cpp:66-73 (strict >, first max wins)
 *
 * The synthetic-data PRNG (orc_normal / orc_uniform) and the bf16 / OCP fp8
 * e4m3 codecs are this build's own specification, restated independently of
 * the product so tests can compare the two bit for bit.
 *
 * Pins (what checks this file; tests/test_cpu_oracle.py):
 *   - end-to-end logits against golden vectors written by importing the
 *     reference's python/model.py (tests/golden/gen_golden.py);
 *   - GEMM against numpy matmul and exact small-integer products;
 *   - LayerNorm / GELU against torch.nn.functional on the CPU;
 *   - attention closed forms (kv_len=1 -> v0, equal keys -> mean of V,
 *     one dominant key -> its V, page-table permutation invariance) and a
 *     dense numpy softmax on tiny inputs;
 *   - e4m3 / bf16 codecs: exhaustive round trips and torch's own casts.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* PRNG spec: counter-based splitmix64; normals by Irwin-Hall(12).           */
/* ------------------------------------------------------------------------ */

static inline uint64_t orc_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

#define ORC_GOLDEN 0x9E3779B97F4A7C15ULL

uint64_t orc_key(uint64_t seed, uint64_t stream) {
  return orc_mix64(seed + ORC_GOLDEN * (orc_mix64(stream + ORC_GOLDEN) | 1ULL));
}

uint64_t orc_u64(uint64_t key, uint64_t i) { return orc_mix64(key + (i + 1) * ORC_GOLDEN); }

/* Exact Irwin-Hall(12) variate: z = (sum of 12 centred 24-bit uniforms) - 6,
 * returned as the exact double 2*S + 12 - 3*2^26 scaled by 2^-25. */
double orc_normal_exact(uint64_t key, uint64_t i) {
  int64_t s = 0;
  for (int j = 0; j < 6; ++j) {
    uint64_t u = orc_u64(key, 6 * i + (uint64_t)j);
    s += (int64_t)(u >> 40) + (int64_t)((u >> 8) & 0xFFFFFFULL);
  }
  int64_t num = 2 * s + 12 - 3 * ((int64_t)1 << 26);
  return (double)num * (1.0 / 33554432.0);
}

void orc_normal_f32(uint64_t seed, uint64_t stream, uint64_t start, int64_t n, double stddev,
                    float* out) {
  uint64_t key = orc_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = (float)(stddev * orc_normal_exact(key, start + (uint64_t)i));
}

void orc_uniform_int(uint64_t seed, uint64_t stream, uint64_t start, int64_t n, int32_t lo,
                     int32_t hi_inclusive, int32_t* out) {
  uint64_t key = orc_key(seed, stream);
  uint64_t range = (uint64_t)((int64_t)hi_inclusive - (int64_t)lo + 1);
  for (int64_t i = 0; i < n; ++i) out[i] = lo + (int32_t)((orc_u64(key, start + (uint64_t)i) >> 11) % range);
}

/* ------------------------------------------------------------------------ */
/* Number formats.                                                           */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fp32 -> bf16, round to nearest even (NaN kept quiet). */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void orc_round_bf16(float* x, int64_t n) {
#pragma omp parallel for schedule(static) if (n > (1 << 20))
  for (int64_t i = 0; i < n; ++i) x[i] = orc_bf16_to_f32(orc_f32_to_bf16(x[i]));
}

/* OCP fp8 e4m3 (bias 7, no infinities, S.1111.111 = NaN, max 448). */
float orc_e4m3_to_f32(uint8_t b) {
  int s = b >> 7, e = (b >> 3) & 0xF, m = b & 7;
  double v;
  if (e == 0xF && m == 7) return NAN;
  if (e == 0) v = ldexp((double)m, -9);
  else v = ldexp(1.0 + m / 8.0, e - 7);
  return (float)(s ? -v : v);
}

/* Round to nearest even on the e4m3 grid, saturating to +-448: scale |f| to
 * units of its binade's quantum (2^(E-3), or 2^-9 below 2^-6) and rint()
 * (round-half-even) in fp64, where the scaling is exact. */
uint8_t orc_f32_to_e4m3(float f) {
  if (isnan(f)) return 0x7F;
  uint8_t sign = signbit(f) ? 0x80 : 0;
  double a = fabs((double)f);
  if (a >= 448.0) return sign | 0x7E;
  if (a < ldexp(1.0, -6)) return sign | (uint8_t)rint(a * 512.0); /* 8 == min normal code */
  int e;
  frexp(a, &e);
  int E = e - 1; /* a in [2^E, 2^(E+1)) */
  double q = rint(ldexp(a, 3 - E));
  if (q == 16.0) { q = 8.0; E += 1; }
  int code = ((E + 7) << 3) | ((int)q - 8);
  if (code > 0x7E) code = 0x7E;
  return sign | (uint8_t)code;
}

/* Per-output-channel absmax quantisation of w [N, K] (fp32): scale[n] =
 * max_k |w[n,k]| / 448 in fp32 (1 for an all-zero row), codes[n,k] =
 * e4m3_rne(w[n,k] / scale[n]) with the quotient rounded to fp32 first.
 * config 5's weight format; rows in parallel. */
void orc_quantize_e4m3_rows(int64_t N, int64_t K, const float* w, uint8_t* codes, float* scale) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const float* r = w + n * K;
    float amax = 0.f;
    for (int64_t k = 0; k < K; ++k) amax = fabsf(r[k]) > amax ? fabsf(r[k]) : amax;
    float sc = amax / 448.0f;
    if (sc == 0.f) sc = 1.0f;
    scale[n] = sc;
    for (int64_t k = 0; k < K; ++k) codes[n * K + k] = orc_f32_to_e4m3(r[k] / sc);
  }
}

/* ------------------------------------------------------------------------ */
/* GEMM with the reference's epilogues.                                      */
/* ------------------------------------------------------------------------ */

/* Y[m,n] = sum_k X[m,k] * W[n,k] * (w_scale ? w_scale[n] : 1) + bias[n]
 * then GELU (erf form) if gelu, then + residual[m,n] if residual.
 * fp64 accumulation.  Follows kernels/linear.cu:15-34 (row-major X.W^T via
 * docs/gemm_layout.md:16-41) with the separate bias/GELU/residual launches of
 * kernels/linear.cu:6-12 and kernels/elementwise.cu:59-73 applied in the
 * order src/transformer.cpp:82-89 uses. */
typedef double orc_v4d __attribute__((vector_size(32)));
enum { kGemmRows = 4, kGemmCols = 8 };

/* acc[i][j] = sum over k = 0 .. K-1, in that order, of x_i[k] * wt[k][j] for
 * kGemmRows rows x_i and the kGemmCols columns packed in wt ([K][8] doubles).
 * Every output keeps one accumulator summed in k order, so the result is the
 * plain loop's bit for bit (a float x float product is exact in fp64); the
 * vectors only run 8 outputs side by side.  Built for AVX2 and for the
 * baseline ISA, chosen at load time. */
__attribute__((target_clones("avx2", "default"))) static void gemm_tile(int K, const float* const* xr,
                                                                         const double* wt,
                                                                         double out[kGemmRows][kGemmCols]) {
  orc_v4d acc[kGemmRows][2];
  for (int i = 0; i < kGemmRows; ++i) acc[i][0] = acc[i][1] = (orc_v4d){0.0, 0.0, 0.0, 0.0};
  for (int k = 0; k < K; ++k) {
    const orc_v4d w0 = *(const orc_v4d*)(wt + 8 * (int64_t)k);
    const orc_v4d w1 = *(const orc_v4d*)(wt + 8 * (int64_t)k + 4);
    for (int i = 0; i < kGemmRows; ++i) {
      const double xv = (double)xr[i][k];
      const orc_v4d xb = {xv, xv, xv, xv};
      acc[i][0] += xb * w0;
      acc[i][1] += xb * w1;
    }
  }
  for (int i = 0; i < kGemmRows; ++i)
    for (int j = 0; j < 4; ++j) {
      out[i][j] = acc[i][0][j];
      out[i][4 + j] = acc[i][1][j];
    }
}

void orc_gemm(int M, int N, int K, const float* X, int ldx, const float* W, int ldw,
              const float* w_scale, const float* bias, int gelu, const float* residual, int ldr,
              double* Y, int ldy) {
  const int nblocks = (N + kGemmCols - 1) / kGemmCols;
#pragma omp parallel
  {
    /* this thread's packed column block: W[n0 .. n0 + 7][0 .. K-1] as [K][8]
     * doubles, zero past N (those columns are never stored) */
    double* wt = (double*)aligned_alloc(64, ((size_t)(K > 0 ? K : 1) * kGemmCols * sizeof(double) + 63) / 64 * 64);
#pragma omp for schedule(dynamic, 1)
    for (int nb = 0; nb < nblocks; ++nb) {
      const int n0 = nb * kGemmCols;
      for (int j = 0; j < kGemmCols; ++j) {
        const float* w = W + (int64_t)(n0 + j) * ldw;
        for (int k = 0; k < K; ++k) wt[(int64_t)k * kGemmCols + j] = n0 + j < N ? (double)w[k] : 0.0;
      }
      for (int m0 = 0; m0 < M; m0 += kGemmRows) {
        const float* xr[kGemmRows];
        for (int i = 0; i < kGemmRows; ++i) xr[i] = X + (int64_t)(m0 + i < M ? m0 + i : M - 1) * ldx;
        double t[kGemmRows][kGemmCols];
        gemm_tile(K, xr, wt, t);
        for (int i = 0; i < kGemmRows && m0 + i < M; ++i)
          for (int j = 0; j < kGemmCols && n0 + j < N; ++j) {
            const int m = m0 + i, n = n0 + j;
            double acc = t[i][j];
            if (w_scale) acc *= (double)w_scale[n];
            if (bias) acc += (double)bias[n];
            if (gelu) acc = 0.5 * acc * (1.0 + erf(acc * 0.70710678118654752440));
            if (residual) acc += (double)residual[(int64_t)m * ldr + n];
            Y[(int64_t)m * ldy + n] = acc;
          }
      }
    }
    free(wt);
  }
}

/* LayerNorm over D with eps, biased variance; kernels/elementwise.cu:21-57,
 * python/model.py:26 (nn.LayerNorm default eps 1e-5).  Two-pass in fp64. */
void orc_layernorm(int M, int D, const float* X, int ldx, const float* g, const float* b,
                   double eps, double* Y, int ldy) {
  for (int m = 0; m < M; ++m) {
    const float* x = X + (int64_t)m * ldx;
    double mean = 0.0, var = 0.0;
    for (int i = 0; i < D; ++i) mean += x[i];
    mean /= D;
    for (int i = 0; i < D; ++i) { double t = x[i] - mean; var += t * t; }
    var /= D;
    double inv = 1.0 / sqrt(var + eps);
    for (int i = 0; i < D; ++i) Y[(int64_t)m * ldy + i] = (x[i] - mean) * inv * g[i] + b[i];
  }
}

/* x[r] = tok_emb[tok[r]] + pos_emb[pos[r]]; kernels/elementwise.cu:7-17. */
void orc_embed(int M, int D, const int32_t* tok, const int32_t* pos, const float* tok_emb,
               const float* pos_emb, double* out) {
  for (int m = 0; m < M; ++m)
    for (int i = 0; i < D; ++i)
      out[(int64_t)m * D + i] = (double)tok_emb[(int64_t)tok[m] * D + i] + (double)pos_emb[(int64_t)pos[m] * D + i];
}

/* Loads element `e` of a pool stored as fp32 (dtype 0) or bf16 (dtype 1). */
static inline double pool_at(const void* pool, int dtype, int64_t e) {
  if (dtype == 0) return (double)((const float*)pool)[e];
  return (double)orc_bf16_to_f32(((const uint16_t*)pool)[e]);
}

/* kpool[page][slot][:] = K[r,:] (rounded to bf16 for a bf16 pool);
 * kernels/attention.cu:7-19. */
void orc_scatter_kv(int M, int D, const double* K, const double* V, void* kpool, void* vpool,
                    int dtype, const int32_t* wpage, const int32_t* woff, int page_size) {
  for (int m = 0; m < M; ++m) {
    int64_t base = ((int64_t)wpage[m] * page_size + woff[m]) * D;
    for (int i = 0; i < D; ++i) {
      if (dtype == 0) {
        ((float*)kpool)[base + i] = (float)K[(int64_t)m * D + i];
        ((float*)vpool)[base + i] = (float)V[(int64_t)m * D + i];
      } else {
        ((uint16_t*)kpool)[base + i] = orc_f32_to_bf16((float)K[(int64_t)m * D + i]);
        ((uint16_t*)vpool)[base + i] = orc_f32_to_bf16((float)V[(int64_t)m * D + i]);
      }
    }
  }
}

/* Causal paged attention, kernels/attention.cu:57-98: row r attends to keys
 * j in [0, row_pos[r]] of its sequence; key j lives in physical page
 * table[j / page_size], slot j % page_size; pools are [P][page][H][hd].
 * Row r's table is block_table + (row_bt ? row_bt[r] : r) * bt_stride.
 * q is read as float (ldq floats per row).  Exact two-pass softmax in fp64
 * (python/model.py:40-44), which the reference's online softmax equals up
 * to rounding. */
void orc_paged_attention(int M, int H, int hd, int page_size, const void* kpool, const void* vpool,
                         int dtype, const int32_t* block_table, int bt_stride, const int32_t* row_bt,
                         const int32_t* row_pos, const float* q, int ldq, double* out, int ldo) {
  const int D = H * hd;
  const double scale = 1.0 / sqrt((double)hd);
#pragma omp parallel
  {
    int cap = 0;
    double* s = NULL;
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (int r = 0; r < M; ++r) {
      for (int h = 0; h < H; ++h) {
        const int32_t* tab = block_table + (int64_t)(row_bt ? row_bt[r] : r) * bt_stride;
        int kv = row_pos[r] + 1;
        if (kv > cap) { cap = kv; s = (double*)realloc(s, sizeof(double) * (size_t)cap); }
        const float* qr = q + (int64_t)r * ldq + h * hd;
        double mx = -INFINITY;
        for (int j = 0; j < kv; ++j) {
          int64_t base = ((int64_t)tab[j / page_size] * page_size + (j % page_size)) * D + (int64_t)h * hd;
          double d = 0.0;
          for (int i = 0; i < hd; ++i) d += (double)qr[i] * pool_at(kpool, dtype, base + i);
          s[j] = d * scale;
          if (s[j] > mx) mx = s[j];
        }
        double l = 0.0;
        for (int j = 0; j < kv; ++j) { s[j] = exp(s[j] - mx); l += s[j]; }
        double* o = out + (int64_t)r * ldo + h * hd;
        for (int i = 0; i < hd; ++i) o[i] = 0.0;
        for (int j = 0; j < kv; ++j) {
          int64_t base = ((int64_t)tab[j / page_size] * page_size + (j % page_size)) * D + (int64_t)h * hd;
          double p = s[j] / l;
          for (int i = 0; i < hd; ++i) o[i] += p * pool_at(vpool, dtype, base + i);
        }
      }
    }
    free(s);
  }
}

/* First index of the maximum (strict >), src/bench_batching.cpp:66-73. */
void orc_argmax_rows(int M, int N, const float* logits, int ld, int32_t* out) {
  for (int m = 0; m < M; ++m) {
    const float* row = logits + (int64_t)m * ld;
    int best = 0;
    float bv = row[0];
    for (int n = 1; n < N; ++n)
      if (row[n] > bv) { bv = row[n]; best = n; }
    out[m] = best;
  }
}

/* ------------------------------------------------------------------------ */
/* Whole forward step, src/transformer.cpp:44-99.                            */
/* ------------------------------------------------------------------------ */

/* Weights, already dequantised to float (bf16 / fp8*scale values exactly).
 * w_scale arrays are NULL when the weights are not fp8 (the scale is then
 * already folded into nothing).  Order of the per-layer pointers follows
 * python/export_weights.py:42-66. */
typedef struct {
  const float *ln1_w, *ln1_b;
  const float *wq, *bq, *wk, *bk, *wv, *bv, *wo, *bo;
  const float *ln2_w, *ln2_b;
  const float *fc1, *b1, *fc2, *b2;
  const float *sq, *sk, *sv, *so, *s1, *s2; /* per-output-channel scales or NULL */
} orc_layer_t;

typedef struct {
  int vocab, d_model, n_heads, head_dim, n_layers, mlp, page_size;
  int act_bf16; /* 1: round GEMM inputs (LN outputs, attention output, GELU output) to bf16 */
  int kv_dtype; /* 0 fp32 pool, 1 bf16 pool */
  const float *tok_emb, *pos_emb, *ln_f_w, *ln_f_b, *lm_head, *lm_scale;
  const orc_layer_t* layers;
} orc_model_t;

static void to_float_rounded(const double* src, float* dst, int64_t n, int round_bf16) {
  for (int64_t i = 0; i < n; ++i) {
    float f = (float)src[i];
    dst[i] = round_bf16 ? orc_bf16_to_f32(orc_f32_to_bf16(f)) : f;
  }
}

/* The step in three parts, so a caller can run it one layer at a time over
 * that layer's pools alone (a 16-layer pool set need not be on the host at
 * once): orc_step_embed forms the residual stream x [M, d] (fp64),
 * orc_step_layer runs layer l on it in place, orc_step_head the final
 * LayerNorm and lm_head.  orc_forward_step is the three in sequence. */
void orc_step_embed(const orc_model_t* mdl, int M, const int32_t* token_ids, const int32_t* positions, double* x) {
  orc_embed(M, mdl->d_model, token_ids, positions, mdl->tok_emb, mdl->pos_emb, x);
}

/* Layer l of src/transformer.cpp:65-90 on x [M, d] in place.  K/V of every
 * row are written into this layer's pools (kpool, vpool) at
 * (wpage[i], woff[i]) before its attention runs, as src/transformer.cpp:75-80
 * orders them; row i's page table is block_table + row_bt[i] * bt_stride. */
void orc_step_layer(const orc_model_t* mdl, int l, int M, double* x, const int32_t* positions,
                    const int32_t* wpage, const int32_t* woff, const int32_t* block_table, int bt_stride,
                    const int32_t* row_bt, void* kpool, void* vpool) {
  const int D = mdl->d_model, F = mdl->mlp, H = mdl->n_heads, hd = mdl->head_dim;
  const int rb = mdl->act_bf16;
  const orc_layer_t* w = &mdl->layers[l];
  double* t = (double*)malloc(sizeof(double) * (size_t)M * D);
  double* kd = (double*)malloc(sizeof(double) * (size_t)M * D);
  double* vd = (double*)malloc(sizeof(double) * (size_t)M * D);
  double* hbuf = (double*)malloc(sizeof(double) * (size_t)M * F);
  float* xf = (float*)calloc((size_t)M * D, sizeof(float));
  float* af = (float*)malloc(sizeof(float) * (size_t)M * (F > D ? F : D));
  float* qf = (float*)malloc(sizeof(float) * (size_t)M * D);
  /* LN1 */
  to_float_rounded(x, xf, (int64_t)M * D, 0);
  orc_layernorm(M, D, xf, D, w->ln1_w, w->ln1_b, 1e-5, t, D);
  to_float_rounded(t, af, (int64_t)M * D, rb);
  /* Q, K, V */
  orc_gemm(M, D, D, af, D, w->wq, D, w->sq, w->bq, 0, NULL, 0, t, D);
  to_float_rounded(t, qf, (int64_t)M * D, 0);
  orc_gemm(M, D, D, af, D, w->wk, D, w->sk, w->bk, 0, NULL, 0, kd, D);
  orc_gemm(M, D, D, af, D, w->wv, D, w->sv, w->bv, 0, NULL, 0, vd, D);
  orc_scatter_kv(M, D, kd, vd, kpool, vpool, mdl->kv_dtype, wpage, woff, mdl->page_size);
  /* attention */
  orc_paged_attention(M, H, hd, mdl->page_size, kpool, vpool, mdl->kv_dtype, block_table, bt_stride, row_bt,
                      positions, qf, D, t, D);
  to_float_rounded(t, af, (int64_t)M * D, rb);
  /* out-projection + residual */
  to_float_rounded(x, xf, (int64_t)M * D, 0);
  orc_gemm(M, D, D, af, D, w->wo, D, w->so, w->bo, 0, xf, D, x, D);
  /* LN2, fc1 + GELU, fc2 + residual */
  to_float_rounded(x, xf, (int64_t)M * D, 0);
  orc_layernorm(M, D, xf, D, w->ln2_w, w->ln2_b, 1e-5, t, D);
  to_float_rounded(t, af, (int64_t)M * D, rb);
  orc_gemm(M, F, D, af, D, w->fc1, D, w->s1, w->b1, 1, NULL, 0, hbuf, F);
  to_float_rounded(hbuf, af, (int64_t)M * F, rb);
  orc_gemm(M, D, F, af, F, w->fc2, F, w->s2, w->b2, 0, xf, D, x, D);
  free(t); free(kd); free(vd); free(hbuf); free(xf); free(af); free(qf);
}

/* Final LayerNorm and lm_head (no bias, python/model.py:61): logits [M, vocab]. */
void orc_step_head(const orc_model_t* mdl, int M, const double* x, double* logits) {
  const int D = mdl->d_model;
  double* t = (double*)malloc(sizeof(double) * (size_t)M * D);
  float* xf = (float*)calloc((size_t)M * D, sizeof(float));
  float* af = (float*)malloc(sizeof(float) * (size_t)M * D);
  to_float_rounded(x, xf, (int64_t)M * D, 0);
  orc_layernorm(M, D, xf, D, mdl->ln_f_w, mdl->ln_f_b, 1e-5, t, D);
  to_float_rounded(t, af, (int64_t)M * D, mdl->act_bf16);
  orc_gemm(M, mdl->vocab, D, af, D, mdl->lm_head, D, mdl->lm_scale, NULL, 0, NULL, 0, logits, mdl->vocab);
  free(t); free(xf); free(af);
}

/* One flattened continuous-batch step, src/transformer.cpp:44-99: rows are
 * (token_ids[i], positions[i]); layer l uses the pools kpools[l], vpools[l].
 * logits is [M, vocab] (double). */
void orc_forward_step(const orc_model_t* mdl, int M, const int32_t* token_ids, const int32_t* positions,
                      const int32_t* wpage, const int32_t* woff, const int32_t* block_table, int bt_stride,
                      const int32_t* row_bt, void* const* kpools, void* const* vpools, double* logits) {
  double* x = (double*)malloc(sizeof(double) * (size_t)M * mdl->d_model);
  orc_step_embed(mdl, M, token_ids, positions, x);
  for (int l = 0; l < mdl->n_layers; ++l)
    orc_step_layer(mdl, l, M, x, positions, wpage, woff, block_table, bt_stride, row_bt, kpools[l], vpools[l]);
  orc_step_head(mdl, M, x, logits);
  free(x);
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Threads for the following calls (bench.py times a 1-core and an all-core
 * sample); returns the previous count. */
int orc_set_num_threads(int n) {
#ifdef _OPENMP
  const int old = omp_get_max_threads();
  if (n > 0) omp_set_num_threads(n);
  return old;
#else
  (void)n;
  return 1;
#endif
}
