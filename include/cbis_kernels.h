/*
 * cbis_kernels.h -- C-ABI of the MI355X (gfx950) kernels behind the per-step
 * transformer forward.
 *
 * This is the drop-in boundary.  In the reference the kernels sit behind
 * seven C++ launchers taking raw device pointers, int dims and a stream:
 *   include/linear.hpp:9-11       linear_forward          (cuBLAS SGEMM + bias)
 *   include/elementwise.hpp:6-8   embed_lookup_add
 *   include/elementwise.hpp:12-13 layernorm_forward
 *   include/elementwise.hpp:15-18 gelu_forward
 *   include/elementwise.hpp:20-21 residual_add
 *   include/attention.hpp:8-12    scatter_kv_to_cache
 *   include/attention.hpp:29-33   fused_paged_causal_attention
 * Each has an extern "C" twin below with the same argument meaning (minus
 * the cuBLAS handle).  Beside them are the descriptor entry points the
 * runtime uses: the MFMA GEMM with fused epilogues (bias, GELU, residual,
 * K/V page scatter; fp32, bf16 and fp8-e4m3 weights), split-KV paged decode
 * attention with a caller-provided workspace, MFMA prefill attention over
 * paged K/V, LayerNorm with a bf16 output, device argmax and synthetic fills.
 *
 * Conventions: every pointer argument is a device pointer unless stated;
 * layouts are row-major; weights use nn.Linear's [out, in] layout
 * (docs/gemm_layout.md:16-41); K/V pools are [pages][page_size][heads][head_dim].
 * Entry points are stream-ordered, allocate nothing, and return 0 on success
 * or a non-zero cbis_status; cbis_last_error() then holds a message (per
 * thread).  Every buffer a call (or a descriptor it reads) points to -- row
 * lists, page tables, workspaces included -- must stay allocated and
 * unmodified by other work until the launched kernels finish on the stream:
 * the kernels read them asynchronously.  They never exit() (the reference's CUDA_CHECK does,
 * include/cuda_check.hpp:7-15).
 */
#ifndef CBIS_KERNELS_H
#define CBIS_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* cbis_stream_t; /* a hipStream_t; NULL is the default stream */

enum cbis_dtype { CBIS_F32 = 0, CBIS_BF16 = 1, CBIS_FP8E4M3 = 2 };

enum cbis_status {
  CBIS_OK = 0,
  CBIS_ERR_INVALID = 1,     /* bad argument (null pointer, size, alignment) */
  CBIS_ERR_UNSUPPORTED = 2, /* shape/dtype combination this build has no kernel for */
  CBIS_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  CBIS_ERR_HIP = 4          /* the HIP runtime reported an error */
};

/* Message for the last non-zero status returned on this thread. */
const char* cbis_last_error(void);

/* ----------------------------------------------------------------------- */
/* Reference-signature entry points (fp32 throughout).                      */
/* ----------------------------------------------------------------------- */

/* Y[T,out] = X[T,in] . W[out,in]^T + b (b may be NULL).
 * Replaces linear_forward, include/linear.hpp:9-11 / kernels/linear.cu:15-34. */
int cbis_linear_forward(const float* X, const float* W, const float* b, float* Y, int T,
                        int in_features, int out_features, cbis_stream_t stream);

/* out[r] = tok_emb[token_ids[r]] + pos_emb[positions[r]].
 * Replaces embed_lookup_add, include/elementwise.hpp:6-8.  Like the reference
 * the tables' sizes are not known here and ids are trusted, except that a
 * negative id gives an all-NaN row instead of a read before the table. */
int cbis_embed_lookup_add(const int* token_ids, const int* positions, const float* tok_emb,
                          const float* pos_emb, float* out, int T, int d_model, cbis_stream_t stream);

/* Y = LayerNorm(X) * gamma + beta, eps 1e-5.
 * Replaces layernorm_forward, include/elementwise.hpp:12-13. */
int cbis_layernorm_forward(const float* X, const float* gamma, const float* beta, float* Y, int T,
                           int d_model, cbis_stream_t stream);

/* In-place exact-erf GELU.  Replaces gelu_forward, include/elementwise.hpp:15-18. */
int cbis_gelu_forward(float* X, int T, int width, cbis_stream_t stream);

/* X += Y.  Replaces residual_add, include/elementwise.hpp:20-21. */
int cbis_residual_add(float* X, const float* Y, int T, int width, cbis_stream_t stream);

/* Copies row r of K/V into slot (write_page[r], write_offset[r]) of the pools.
 * Replaces scatter_kv_to_cache, include/attention.hpp:8-12. */
int cbis_scatter_kv_to_cache(const float* K_proj, const float* V_proj, float* k_pages, float* v_pages,
                             const int* write_page, const int* write_offset, int total_rows, int d_model,
                             int page_size, int n_heads, int head_dim, cbis_stream_t stream);

/* Causal paged attention with the reference's per-row page table
 * row_page_table[total_rows, pages_per_seq]; kv_len = row_query_pos[r] + 1.
 * Replaces fused_paged_causal_attention, include/attention.hpp:29-33
 * (kernels/attention.cu:57-127).  Needs no workspace.  page_size 16 runs the
 * wave64 decode kernel in a single pass per (row, head block); any other
 * page_size > 0 runs a one-wave-per-(row, head) kernel whose lanes take one
 * key each (the reference takes page_size at run time).  head_dim 32, as the
 * reference's one-warp-per-(row, head) kernel requires; any n_heads (the
 * reference's grid(total_rows, n_heads)). */
int cbis_fused_paged_causal_attention(const float* Q_proj, const float* k_pages, const float* v_pages,
                                      const int* row_page_table, const int* row_query_pos, float* attn_out,
                                      int total_rows, int n_heads, int head_dim, int page_size,
                                      int pages_per_seq, cbis_stream_t stream);

/* ----------------------------------------------------------------------- */
/* GEMM: Y = epilogue(X . W^T) on MFMA.                                     */
/* ----------------------------------------------------------------------- */

enum cbis_epilogue { CBIS_EPI_NONE = 0, CBIS_EPI_GELU = 1 };

typedef struct cbis_gemm_desc {
  int M, N, K;
  int x_dtype;           /* CBIS_F32 or CBIS_BF16 */
  const void* X;         /* [M, K], row stride ldx elements */
  int64_t ldx;
  int w_dtype;           /* CBIS_F32 (needs x F32), CBIS_BF16 or CBIS_FP8E4M3 (need x BF16) */
  const void* W;         /* [N, K], row stride ldw elements */
  int64_t ldw;
  const float* w_scale;  /* [N] per-output-channel scale (fp8 only), else NULL */
  const float* bias;     /* [N] or NULL */
  int epilogue;          /* cbis_epilogue, applied after scale and bias */
  const float* residual; /* [M, N] fp32 added last (may alias Y), or NULL */
  int64_t ldr;
  int y_dtype;           /* CBIS_F32 or CBIS_BF16 */
  void* Y;               /* [M, N] (columns >= kv_col0 excluded when scattering) */
  int64_t ldy;
  /* Optional K/V page scatter (the fused form of scatter_kv_to_cache):
   * columns [kv_col0, kv_col0 + kv_width) go to k_pool and the next kv_width
   * to v_pool at slot (write_page[r], write_offset[r]).  kv_pool NULL = off. */
  int kv_col0, kv_width, kv_dtype, page_size;
  void* k_pool;
  void* v_pool;
  const int* write_page;
  const int* write_offset;
  /* Optional split-K workspace (fp32 partials).  With enough of it the
   * library splits K for problems whose output tiles alone cannot fill the
   * GPU; NULL / too small runs without splitting. */
  void* workspace;
  size_t workspace_bytes;
} cbis_gemm_desc;

/* Bytes of workspace that let cbis_gemm use its preferred split-K for this
 * descriptor (0 when it does not split). */
size_t cbis_gemm_workspace_size(const cbis_gemm_desc* d);

int cbis_gemm(const cbis_gemm_desc* d, cbis_stream_t stream);

/* Bytes of workspace that let cbis_gemm_layernorm split K as it prefers: as
 * cbis_gemm_workspace_size, and for decode-sized calls (M <= 64), whose
 * reduce it folds into its LayerNorm kernel, the skinny kernel's split too. */
size_t cbis_gemm_layernorm_workspace_size(const cbis_gemm_desc* d);
/* cbis_gemm, then a row LayerNorm of its fp32 output Y [M, N] (gamma / beta
 * of N values, eps) into ln_out (fp32 or bf16, row pitch ld_ln): the step's
 * "x += h . W2^T + b2; xn = LayerNorm(x)" (src/transformer.cpp:88-89 with the
 * next layer's layernorm_forward at :69, or the final one at :92; likewise the
 * out-projection's :81-82 with :84).  When the
 * GEMM splits K the split reduce and the LayerNorm run as one kernel; the
 * results are those of cbis_gemm followed by cbis_layernorm.  Needs Y fp32
 * without K/V scatter, N a multiple of 4 and <= 8192. */
int cbis_gemm_layernorm(const cbis_gemm_desc* d, const float* ln_gamma, const float* ln_beta, float eps,
                        int ln_dtype, void* ln_out, int64_t ld_ln, cbis_stream_t stream);

/* lm_head fused with the greedy rule (no counterpart kernel in the reference,
 * which copies the [M, vocab] logits to the host and scans each row,
 * src/transformer.cpp:93-97 with src/bench_batching.cpp:66-73):
 * next_token[r] = the first index of the maximum of row r of
 * Y = X . W^T * w_scale + bias (strict >, as argmax_row), and, when margin is
 * not NULL, margin[r] = that maximum minus the largest value at any other
 * index (0 for a tied maximum).  NaN logits never win, except at column 0:
 * the reference's scan starts from the row's first value, so a NaN there makes
 * the token 0 (its margin is then +inf, or NaN when another logit is +inf).
 * The kernels that reduce in their epilogue
 * (M <= 64, and bf16 weights on the wave-specialised tilings) never store Y;
 * the others store the logits in d->Y (when it is an fp32 [M, N] buffer) or
 * the workspace and reduce them.  The epilogue must be scale and bias only
 * (no GELU, residual or K/V scatter).  workspace: 16-byte aligned, at least
 * cbis_gemm_argmax_workspace_size(d) bytes. */
size_t cbis_gemm_argmax_workspace_size(const cbis_gemm_desc* d);
int cbis_gemm_argmax(const cbis_gemm_desc* d, int* next_token, float* margin, void* workspace,
                     size_t workspace_bytes, cbis_stream_t stream);

/* cbis_gemm_argmax of LayerNorm(x): the final layernorm_forward + lm_head +
 * argmax of src/transformer.cpp:92-93 and src/bench_batching.cpp:66-73 in one
 * call, with cbis_layernorm_gemm's rule for where the LayerNorm runs (inside
 * the skinny GEMM for M <= 64 and K <= 512, else cbis_layernorm into d->X
 * first); tokens and margins as cbis_gemm_argmax's, bit for bit. */
int cbis_layernorm_gemm_argmax(const cbis_gemm_desc* d, const float* x, int64_t ldx, const float* ln_gamma,
                               const float* ln_beta, float eps, int* next_token, float* margin, void* workspace,
                               size_t workspace_bytes, cbis_stream_t stream);

/* ----------------------------------------------------------------------- */
/* Paged attention.                                                          */
/* ----------------------------------------------------------------------- */

typedef struct cbis_attn_desc {
  int n_rows;              /* rows to process (entries of `rows`, or 0..n_rows-1) */
  const int* rows;         /* [n_rows] row ids into q/out/row_pos/row_bt, or NULL */
  int n_heads, head_dim, page_size;
  int q_dtype;             /* CBIS_F32 or CBIS_BF16 */
  const void* q;           /* [*, n_heads*head_dim], row stride ldq elements */
  int64_t ldq;
  int kv_dtype;            /* CBIS_F32 or CBIS_BF16 */
  const void* k_pool;      /* [num_pages, page_size, n_heads, head_dim] */
  const void* v_pool;
  int num_pages;           /* pool size; page ids are clamped to it */
  const int* block_table;  /* [*, bt_stride] physical page ids */
  int64_t bt_stride;
  const int* row_bt;       /* row -> block_table row, or NULL (row r uses row r) */
  const int* row_pos;      /* row -> query position; kv_len = pos + 1 */
  int out_dtype;           /* CBIS_F32 or CBIS_BF16 */
  void* out;               /* [*, n_heads*head_dim], row stride ldo elements */
  int64_t ldo;
  int max_kv_len;          /* host upper bound of pos+1 over the rows */
  int split_tokens;        /* tokens per split-KV chunk, 0 = auto; a multiple of
                              page_size, else the call fails with CBIS_ERR_INVALID */
  void* workspace;         /* fp32 partials when a row needs more than one split */
  size_t workspace_bytes;
  int tile_pages;          /* prefill tiles: 0 = [n_tiles][4]; 8 = [n_tiles][12], the
                              tile's first 8 page ids appended (see
                              cbis_paged_prefill_attention) */
} cbis_attn_desc;

/* Bytes of workspace cbis_paged_attention needs for this descriptor (0 when
 * every row fits one split).  Resolves split_tokens = 0 the same way. */
size_t cbis_paged_attention_workspace_size(const cbis_attn_desc* d);

/* Split-KV decode attention: any set of rows, each with its own kv_len. */
int cbis_paged_attention(const cbis_attn_desc* d, cbis_stream_t stream);

/* Decode attention fused with the out-projection that follows it: the
 * attention, linear_forward and residual_add of src/transformer.cpp:78-83
 * in one launch (one launch per layer fewer on small decode steps).  For
 * d's rows, as cbis_paged_attention computes them, but in one
 * pass per row (split_tokens, workspace and out are not used):
 * Y[r, :] = attn(r) . W^T (* w_scale) (+ bias) (+ residual[r, :]) with the
 * attention output rounded to proj->x_dtype first (fp32 or bf16), i.e.
 * cbis_gemm over the attention output that cbis_paged_attention would have
 * stored, summed in another order.  proj: N = K = n_heads * head_dim, W fp32
 * or bf16 (16-byte aligned rows), fp32 Y (may alias residual), no GELU, no
 * K/V scatter; X and M are not read.  Supported: one head block
 * (n_heads * head_dim <= 256 with fp32 K/V, <= 512 with bf16), that width
 * a multiple of 64 and at most 256 with fp32 W (512 with bf16);
 * CBIS_ERR_UNSUPPORTED otherwise.  Meant for short rows: a row's keys are
 * read by n_heads * head_dim / 64 workgroups, each in one pass. */
int cbis_paged_attention_proj(const cbis_attn_desc* d, const cbis_gemm_desc* proj, cbis_stream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc):
 * cbis_paged_attention with the split-KV partials in a library-owned static
 * device buffer of CBIS_ATTN_STATIC_SCRATCH_BYTES per GPU instead of a caller
 * workspace (d->workspace / workspace_bytes are ignored); same kernels, same
 * results.  It calls no hipMalloc / hipFree.  A call whose partials
 * (cbis_paged_attention_workspace_size) exceed the buffer fails with
 * CBIS_ERR_WORKSPACE.  Every call on one GPU shares that GPU's buffer: calls
 * that overlap on one GPU (on different streams, or from several threads)
 * race and may return wrong results; calls ordered on one stream do not.  The
 * buffer keeps the last call's contents; nothing in it needs to start at
 * zero.  The first call on a device looks up the buffer's address there. */
#define CBIS_ATTN_STATIC_SCRATCH_BYTES ((size_t)32 << 20)
int cbis_paged_attention_static(const cbis_attn_desc* d, cbis_stream_t stream);

/* Rows per prefill tile, at most. */
#define CBIS_PREFILL_TILE_ROWS 64

/* Prefill attention on MFMA for query tiles of <= CBIS_PREFILL_TILE_ROWS
 * consecutive rows of one sequence.  tiles is a device array [n_tiles][4] of
 * {first_row, n_valid_rows, block_table_row, first_position}; row i of a tile
 * has position first_position + i and attends causally to keys [0, position].
 * With d->tile_pages = 8 a tile is 12 ints: those 4, then for k = 0..7 the
 * block-table entry of page min(16 k, kv_end - 1) / 16 of its row, kv_end =
 * min(first_position + n_valid_rows, bt_stride * page_size) (the pages the
 * tile's first key blocks read, so their loads need no block-table read
 * first; same results).  Rows of a tile past CBIS_PREFILL_TILE_ROWS are not
 * computed.  d->rows / row_bt / row_pos / max_kv_len / split_tokens /
 * workspace are ignored.  Supports bf16 K/V, head_dim 32, page_size 16. */
int cbis_paged_prefill_attention(const cbis_attn_desc* d, int n_tiles, const int* tiles,
                                 cbis_stream_t stream);

/* A step's attention in two launches: cbis_paged_attention over d's rows (the
 * single decode rows) then cbis_paged_prefill_attention over the tiles, with
 * the decode rows' split merge run inside the prefill launch instead of a
 * launch of its own.  Results are those of the two calls.  The forms of
 * src/transformer.cpp:77-79 (fused_paged_causal_attention over every row of
 * the step) the runner uses.  Either part may be empty (n_rows / n_tiles 0). */
int cbis_paged_attention_mixed(const cbis_attn_desc* d, int n_tiles, const int* tiles, cbis_stream_t stream);

/* ----------------------------------------------------------------------- */
/* Row ops.                                                                  */
/* ----------------------------------------------------------------------- */

/* out[r,:] = tok_emb[token_ids[r],:] + pos_emb[positions[r],:] (fp32 out);
 * embeddings fp32 or bf16.  A row whose token id is outside [0, vocab) or
 * position outside [0, max_pos) reads nothing and comes out all NaN. */
int cbis_embed(int T, int d_model, const int* token_ids, const int* positions, int emb_dtype,
               const void* tok_emb, const void* pos_emb, int vocab, int max_pos, float* out,
               cbis_stream_t stream);

/* cbis_embed where a row's token may come from the device (no reference
 * counterpart: it lets a decode step take its input tokens from the step
 * before without a round trip through the host).  Row r uses token
 * src_tokens[token_src[r]] when token_src[r] >= 0, else token_ids[r];
 * token_src and src_tokens are both NULL (plain cbis_embed) or both set.
 * The same rule for ids out of range applies to the token used.
 * stage_bytes > 0 (a multiple of 16, both buffers 16-byte aligned, T > 0)
 * also copies stage_src to stage_dst within the same launch: a caller that
 * keeps a step's metadata in device-visible pinned host memory has it on the
 * device for the kernels after this one without a separate copy.  The
 * indices read here (token_ids, token_src, positions) may point into that
 * host memory; the copy is not visible to this launch itself. */
int cbis_embed_from(int T, int d_model, const int* token_ids, const int* token_src, const int* src_tokens,
                    const int* positions, int emb_dtype, const void* tok_emb, const void* pos_emb, int vocab,
                    int max_pos, float* out, const void* stage_src, void* stage_dst, size_t stage_bytes,
                    cbis_stream_t stream);

/* Row LayerNorm of fp32 X into fp32 or bf16 Y. */
int cbis_layernorm(int T, int d_model, const float* X, int64_t ldx, const float* gamma, const float* beta,
                   float eps, int y_dtype, void* Y, int64_t ldy, cbis_stream_t stream);

/* Y = LayerNorm(x) . W^T with d's epilogue: cbis_layernorm of x [M, K] (fp32,
 * row stride ldx; gamma, beta [K]) into d->X as d->x_dtype, then cbis_gemm(d),
 * the layernorm_forward + linear_forward of src/transformer.cpp:69-72 (and
 * :84-85) in one call.  Decode-sized calls with short rows (the skinny path:
 * M <= 64; K <= 512; x, gamma, beta 16-byte aligned, ldx % 4 == 0) form the
 * normalised rows inside the GEMM instead (one launch, X not written); both
 * ways give the same Y bit for bit.  d->X must be a [M, K] buffer of
 * d->x_dtype (row stride d->ldx). */
int cbis_layernorm_gemm(const cbis_gemm_desc* d, const float* x, int64_t ldx, const float* ln_gamma,
                        const float* ln_beta, float eps, cbis_stream_t stream);

/* out[r] = first index of the maximum of logits[r, 0:N] (strict >), the
 * greedy rule of src/bench_batching.cpp:66-73, NaN included: a NaN at column
 * 0 gives 0 (the scan's first value is never displaced), NaN elsewhere never
 * wins. */
int cbis_argmax_rows(int T, int N, const float* logits, int64_t ld, int* out, cbis_stream_t stream);

/* ----------------------------------------------------------------------- */
/* Synthetic data.                                                           */
/* ----------------------------------------------------------------------- */

/* dst[i] = std * z(seed, stream_id, start + i), z the exact Irwin-Hall(12)
 * variate of the counter-based splitmix64 generator; stored as fp32 or bf16
 * (round to nearest even).  Bit-reproducible on the host. */
int cbis_fill_normal_exact(void* dst, int dtype, int64_t n, uint64_t seed, uint64_t stream_id,
                           uint64_t start, float std, cbis_stream_t stream);

/* ---- Tiered-cache block movement -------------------------------------- */
/* Gathers whole pages of a paged K/V allocation laid out
 * [n_layers][2 (K, V)][max_pages][page_bytes] (PagedKVCache's single device
 * allocation) into block-major staging [n_pages][n_layers][2][page_bytes]:
 * block b = every layer's K and V page pages[b], in the byte order of one
 * block of the reference's tiered cache.  Replaces read_raw_from_gpu
 * (src/tiered_kv_manager.cpp:69-82, 2 * n_layers copies per block) with one
 * launch per batch.  pages: device int32[n_pages]; page ids outside
 * [0, max_pages) are skipped (callers validate them); page_bytes a multiple
 * of 16; staging / pools 16-byte aligned. */
int cbis_kv_pages_gather(void* staging, const void* pools, int n_layers, int max_pages, int64_t page_bytes,
                         const int* pages, int n_pages, cbis_stream_t stream);
/* The inverse: staging block b -> page pages[b] of every layer's K and V
 * pool (write_raw_to_gpu, src/tiered_kv_manager.cpp:84-98). */
int cbis_kv_pages_scatter(void* pools, const void* staging, int n_layers, int max_pages, int64_t page_bytes,
                          const int* pages, int n_pages, cbis_stream_t stream);

/* Fast N(0, std) fill for large synthetic activations / K/V pools:
 * Box-Muller over a 32-bit hash of (seed, index), fp32 or bf16. */
int cbis_fill_normal_fast(void* dst, int dtype, int64_t n, uint64_t seed, float std, cbis_stream_t stream);

/* dst[i] = src[i] stored as fp32 or bf16 (round to nearest even). */
int cbis_convert_f32(void* dst, int dst_dtype, const float* src, int64_t n, cbis_stream_t stream);

/* Per-output-channel OCP fp8 e4m3 quantisation of an fp32 [N, K] weight:
 * scale[n] = absmax(src[n,:]) / 448 (fp32; 1 for an all-zero row),
 * codes[n,k] = RNE_e4m3(src[n,k] / scale[n]). */
int cbis_quantize_fp8_rows(uint8_t* codes, float* scale, const float* src, int N, int K, cbis_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CBIS_KERNELS_H */
