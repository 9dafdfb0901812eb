// TransformerRunner::forward_step -- one flattened continuous-batch step,
// src/transformer.cpp:44-99, on the gfx950 kernels of cbis_kernels.h.
//
// Differences from the reference's step that keep its contract:
//  * per-step metadata (token ids, positions, write slots, a compact block
//    table per distinct sequence instead of a kPagesPerSeq-wide copy per row,
//    decode-row list, prefill tiles) is packed into one block of pinned,
//    device-visible host memory that the step's embed launch copies to the
//    device on its way (no copy command on the stream); a greedy step's
//    argmax stores its tokens straight into pinned host memory;
//  * per layer: LayerNorm -> one fused QKV GEMM whose epilogue adds the bias
//    and scatters K/V into their page slots (scatter-before-attention order
//    of src/transformer.cpp:75-80 kept) -> split-KV decode attention for
//    single rows and MFMA prefill attention for runs of consecutive rows of
//    one sequence -> out-projection GEMM with bias + residual epilogue ->
//    LayerNorm -> fc1 GEMM with bias + GELU -> fc2 GEMM with bias + residual;
//  * steps whose shape repeats replay a captured HIP graph;
//  * forward_step_greedy runs lm_head fused with the row argmax and top-2
//    margin on the device (no logits stored where the GEMM reduces them).
#include <algorithm>
#include <chrono>
#include <cstring>
#include <unordered_map>

#include "runtime.hpp"

namespace cbis {

namespace {
constexpr int kMinPrefillRun = 8;   // runs shorter than this use the decode kernel
constexpr int kTileRows = CBIS_PREFILL_TILE_ROWS;  // query rows per prefill tile
constexpr int kTileInts = 12;  // a prefill tile's descriptor with its first 8 page ids (tile_pages = 8)
constexpr size_t kMaxGraphs = 64;
size_t align_ints(size_t n) { return (n + 3) & ~(size_t)3; }
}  // namespace

TransformerRunner::TransformerRunner(const ModelWeights& weights, PagedKVCache& cache, int max_total_rows)
    : w_(weights), cache_(cache), cfg_(weights.cfg), max_rows_(max_total_rows) {
  cfg_.validate();
  if (max_total_rows <= 0) throw std::invalid_argument("TransformerRunner: max_total_rows must be > 0");
  if (cache.num_layers() != cfg_.n_layers || cache.n_heads() != cfg_.n_heads || cache.head_dim() != cfg_.head_dim ||
      cache.page_size() != cfg_.page_size || cache.kv_dtype() != cfg_.kv_dtype)
    throw std::invalid_argument("TransformerRunner: cache geometry does not match the model config");
  if (!cache.has_device()) throw std::invalid_argument("TransformerRunner: cache has no device pools");
  // The attention kernels are built for head_dim 32 (any head count).
  if (cfg_.head_dim != 32) throw std::invalid_argument("TransformerRunner: attention needs head_dim 32");
  hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
  const size_t R = max_total_rows, D = cfg_.d_model, F = cfg_.mlp, V = cfg_.vocab;
  const size_t ae = dtype_size(cfg_.act_dtype());
  // cbis_paged_attention_proj's limits: one head block (256 fp32 / 512 bf16
  // K/V columns), a multiple of 64, at most 256 fp32 / 512 bf16 weight columns.
  attn_proj_ok_ = D % 64 == 0 && D <= (cfg_.kv_dtype == CBIS_F32 ? 256u : 512u) &&
                  (cfg_.weight_dtype == CBIS_F32 ? D <= 256 : cfg_.weight_dtype == CBIS_BF16 && D <= 512);
  for (StepBuf& b : bufs_) {
    hip_check(hipEventCreate(&b.ev_start), "hipEventCreate");
    hip_check(hipEventCreate(&b.ev_stop), "hipEventCreate");
    // Greedy results: a step's M tokens, then its M margins right after
    // them, stored by the argmax launch straight into host memory (a copy
    // command after the step would cost more than the step's last kernel).
    hip_check(hipHostMalloc((void**)&b.h_next, R * 8, hipHostMallocMapped | hipHostMallocCoherent),
              "hipHostMalloc next");
    hip_check(hipHostGetDevicePointer((void**)&b.d_next, b.h_next, 0), "hipHostGetDevicePointer next");
  }
  hip_check(hipMalloc((void**)&d_x_, R * D * 4), "hipMalloc x");
  hip_check(hipMalloc(&d_xn_, R * D * ae), "hipMalloc xn");
  hip_check(hipMalloc((void**)&d_q_, R * D * 4), "hipMalloc q");
  hip_check(hipMalloc(&d_attn_, R * D * ae), "hipMalloc attn");
  hip_check(hipMalloc(&d_h_, R * F * ae), "hipMalloc h");
  hip_check(hipMalloc((void**)&d_logits_, R * V * 4), "hipMalloc logits");
  // Split-KV partials: the automatic split keeps rows * splits <= 2048 + rows.
  ws_bytes_ = (2048 + R) * (size_t)cfg_.n_heads * (cfg_.head_dim + 4) * 4;
  hip_check(hipMalloc(&d_ws_, ws_bytes_), "hipMalloc attention workspace");
  // Split-K workspace: the largest any of the step's GEMM shapes asks for at
  // any row count up to max_total_rows (through cbis_gemm_layernorm, whose
  // decode-sized calls split too).
  const int shapes[5][2] = {{3 * (int)D, (int)D}, {(int)D, (int)D}, {(int)F, (int)D}, {(int)D, (int)F}, {(int)V, (int)D}};
  cbis_gemm_desc q = {};
  q.x_dtype = cfg_.act_dtype();
  q.w_dtype = cfg_.weight_dtype;
  q.W = w_.lm_head;  // any weight pointer of the arena: only its alignment is inspected
  for (int m = 1; m <= max_total_rows; ++m)
    for (const auto& sh : shapes) {
      q.M = m; q.N = sh[0]; q.K = sh[1]; q.ldw = sh[1];
      gemm_ws_bytes_ = std::max(gemm_ws_bytes_, cbis_gemm_layernorm_workspace_size(&q));
    }
  if (gemm_ws_bytes_) hip_check(hipMalloc(&d_gemm_ws_, gemm_ws_bytes_), "hipMalloc gemm workspace");
  // Greedy lm_head partials (the logits buffer serves paths that store them).
  q.N = (int)V; q.K = (int)D; q.ldw = (int)D;
  q.Y = d_logits_; q.y_dtype = CBIS_F32; q.ldy = (int)V;
  for (int m = 1; m <= max_total_rows; ++m) {
    q.M = m;
    amax_ws_bytes_ = std::max(amax_ws_bytes_, cbis_gemm_argmax_workspace_size(&q));
  }
  if (amax_ws_bytes_) hip_check(hipMalloc(&d_amax_ws_, amax_ws_bytes_), "hipMalloc argmax workspace");
}

TransformerRunner::~TransformerRunner() {
  if (stream_) (void)hipStreamSynchronize(stream_);  // queued steps still use the buffers
  for (auto& g : graphs_) (void)hipGraphExecDestroy(g.second.exec);
  if (stream_) (void)hipStreamDestroy(stream_);
  for (StepBuf& b : bufs_) {
    if (b.ev_start) (void)hipEventDestroy(b.ev_start);
    if (b.ev_stop) (void)hipEventDestroy(b.ev_stop);
    if (b.h_next) (void)hipHostFree(b.h_next);
    if (b.d_meta) (void)hipFree(b.d_meta);
    if (b.h_meta) (void)hipHostFree(b.h_meta);
  }
  (void)hipFree(d_x_); (void)hipFree(d_xn_); (void)hipFree(d_q_); (void)hipFree(d_attn_);
  (void)hipFree(d_h_); (void)hipFree(d_logits_);
  (void)hipFree(d_ws_);
  if (d_amax_ws_) (void)hipFree(d_amax_ws_);
  if (d_gemm_ws_) (void)hipFree(d_gemm_ws_);
}

void TransformerRunner::prepare(int b, const int* tok, const int* pos, const int* seq, const int* src, int M) {
  if (M > max_rows_) throw std::runtime_error("forward_step: total_rows exceeds max_total_rows");
  for (int i = 0; i < M; ++i) {
    if (src && src[i] >= 0) {
      if (src[i] >= prev_greedy_rows_)
        throw std::out_of_range("enqueue_greedy: token_src beyond the previous greedy step's rows");
    } else if (tok[i] < 0 || tok[i] >= cfg_.vocab) {
      throw std::out_of_range("forward_step: token id out of range");
    }
    if (pos[i] < 0 || pos[i] >= cfg_.max_seq) throw std::out_of_range("forward_step: position out of range");
  }
  std::vector<int> wpage(M), woff(M), rowbt(M);
  std::unordered_map<int, int> index;
  std::vector<int> seqs;
  int width = 1;
  // Slot of every row, as PagedKVCache::resolve_slot (the same exceptions for
  // an unknown sequence or a position past its pages); the page list and
  // table index are looked up once per run of rows of one sequence.
  const int ps = cfg_.page_size;
  const std::vector<int>* pages = nullptr;
  int cur_seq = 0, cur_idx = -1;
  for (int i = 0; i < M; ++i) {
    if (cur_idx < 0 || seq[i] != cur_seq) {
      pages = &cache_.pages(seq[i]);  // throws std::out_of_range for an unknown sequence
      cur_seq = seq[i];
      auto it = index.find(cur_seq);
      if (it == index.end()) {
        it = index.emplace(cur_seq, (int)seqs.size()).first;
        seqs.push_back(cur_seq);
        width = std::max(width, (int)pages->size());
      }
      cur_idx = it->second;
    }
    wpage[i] = pages->at(pos[i] / ps);  // throws like the reference
    woff[i] = pos[i] % ps;
    rowbt[i] = cur_idx;
  }
  // Rows: runs of consecutive positions of one sequence go to the MFMA
  // prefill kernel (bf16 K/V), everything else to the split-KV decode kernel.
  const bool prefill_ok = cfg_.kv_dtype == CBIS_BF16;
  std::vector<int> drows, tiles;
  int max_kv = 1;
  int64_t sum_kv = 0;
  for (int i = 0; i < M;) {
    int j = i + 1;
    while (j < M && seq[j] == seq[i] && pos[j] == pos[j - 1] + 1) ++j;
    if (prefill_ok && j - i >= kMinPrefillRun) {
      const std::vector<int>& pg = cache_.pages(seq[i]);
      for (int r = i; r < j; r += kTileRows) {
        const int nv = std::min(kTileRows, j - r);
        tiles.insert(tiles.end(), {r, nv, rowbt[r], pos[r]});
        // The pages of the tile's first key blocks (tile_pages = 8): page
        // min(16 k, kv_end - 1) / 16, kv_end = pos[r] + nv (within the
        // sequence's pages, so within the step's block-table width).
        const int last = pos[r] + nv - 1;
        for (int k = 0; k < 8; ++k) tiles.push_back(pg[std::min(16 * k, last) / 16]);
      }
    } else {
      for (int r = i; r < j; ++r) {
        drows.push_back(r);
        max_kv = std::max(max_kv, pos[r] + 1);
        sum_kv += pos[r] + 1;
      }
    }
    i = j;
  }
  // Longest rows first: the decode kernel's workgroups are dispatched in row
  // order, so the long rows' splits start early and the short ones fill the
  // tail.
  std::stable_sort(drows.begin(), drows.end(), [&](int x, int y) { return pos[x] > pos[y]; });
  // Likewise the prefill tiles, by their last key (a tile's work grows with
  // it), with the lighter half reversed: when the grid fits one round of
  // resident workgroups, workgroup w and w + grid/2 share a CU, so the
  // heaviest tile shares its CU with the lightest (config 4: 25.5 -> 23.3 us).
  {
    const int nt = (int)tiles.size() / kTileInts;
    std::vector<int> order(nt);
    for (int t = 0; t < nt; ++t) order[t] = t;
    auto last_key = [&](int t) { return tiles[kTileInts * t + 3] + tiles[kTileInts * t + 1]; };
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return last_key(x) > last_key(y); });
    std::reverse(order.begin() + nt / 2, order.end());
    std::vector<int> sorted(tiles.size());
    for (int t = 0; t < nt; ++t) std::copy_n(&tiles[kTileInts * order[t]], kTileInts, &sorted[kTileInts * t]);
    tiles.swap(sorted);
  }
  M_ = M;
  n_decode_ = (int)drows.size();
  n_tiles_ = (int)tiles.size() / kTileInts;
  n_seqs_ = (int)seqs.size();
  bt_width_ = width;
  max_kv_ = (max_kv + 255) / 256 * 256;  // coarse, so steps share split shapes (and graphs)
  // Steps of decode rows only, at most 64 with keys up to 768 (the attention
  // library's one-pass bound for such calls, so the fused launch reads each
  // row's keys as the separate one would): one launch per layer for the
  // attention and the out-projection.
  fused_proj_ = fuse_decode_ && attn_proj_ok_ && tiles.empty() && (int)drows.size() == M && M <= 64 &&
                max_kv_ <= 768;
  // Decode rows in one pass each (no split-KV partials, no merge) when they
  // give at least 1.5 rounds of resident decode workgroups (kDecodeSlots: two
  // per CU, one per row and head block) and no row is more than twice the
  // mean length: the rows go longest first and the pass then fills the GPU
  // to the end (config 4, 768 workgroups: 531 us against 549 with 1408-token
  // splits).  Otherwise splits of about one CU's share of the rows' tokens,
  // rounded up to a power of two (config 5, 16 rows x 32k tokens: 8192-token
  // splits, 256 workgroups: 624 us against 632 with 4096, 639 with 2048 and
  // 649 with the library's 1024), lengthened until the split partials fit the
  // workspace (rows x splits <= 2048 + max_rows).  Calls with less than 2048
  // tokens per CU keep the attention library's own choice.
  {
    constexpr int64_t kDecodeSlots = 512, kCUs = 256;
    const int hpb = cfg_.kv_dtype == CBIS_BF16 ? 16 : 8;
    const int64_t hblocks = (cfg_.n_heads + hpb - 1) / hpb;
    const int64_t rows = (int64_t)drows.size(), units = rows * hblocks;
    split_tokens_ = 0;
    if (rows > 0 && units >= 3 * kDecodeSlots / 2 && (int64_t)max_kv * rows <= 2 * sum_kv) {
      split_tokens_ = 1 << 30;
    } else if (const int64_t share = (sum_kv * hblocks + kCUs - 1) / kCUs;
               rows > 0 && share >= 2048) {
      // A power of two: the split (and with it the step's graph) stays put
      // while the rows grow by a token per step.
      int64_t split = 64;
      while (split < share) split *= 2;
      while (split < max_kv_ && rows * ((max_kv_ + split - 1) / split) > 2048 + max_rows_) split *= 2;
      split_tokens_ = (int)std::min<int64_t>(split, 1 << 30);
    }
  }

  const size_t o_tok = 0, o_pos = o_tok + align_ints(M), o_wp = o_pos + align_ints(M), o_wo = o_wp + align_ints(M),
               o_rb = o_wo + align_ints(M), o_dr = o_rb + align_ints(M), o_ti = o_dr + align_ints(drows.size()),
               o_bt = o_ti + align_ints(tiles.size()), o_src = o_bt + align_ints((size_t)n_seqs_ * width),
               n_ints = o_src + (src ? align_ints(M) : 0);
  const size_t bytes = n_ints * 4;
  StepBuf& sb = bufs_[b];
  if (bytes > sb.cap) {
    // The captured graphs name the old buffers; a step still queued on the
    // other buffers may be running one of them.
    hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    for (auto& g : graphs_) (void)hipGraphExecDestroy(g.second.exec);
    graphs_.clear();
    if (sb.d_meta) hip_check(hipFree(sb.d_meta), "hipFree meta");
    if (sb.h_meta) hip_check(hipHostFree(sb.h_meta), "hipHostFree meta");
    sb.d_meta = sb.h_meta = sb.hd_meta = nullptr;
    sb.cap = std::max(bytes, (size_t)1 << 20) * 2;
    hip_check(hipMalloc((void**)&sb.d_meta, sb.cap), "hipMalloc meta");
    hip_check(hipHostMalloc((void**)&sb.h_meta, sb.cap, hipHostMallocMapped | hipHostMallocCoherent),
              "hipHostMalloc meta");
    hip_check(hipHostGetDevicePointer((void**)&sb.hd_meta, sb.h_meta, 0), "hipHostGetDevicePointer meta");
  }
  int* h = (int*)sb.h_meta;
  std::memcpy(h + o_tok, tok, M * 4);
  std::memcpy(h + o_pos, pos, M * 4);
  std::memcpy(h + o_wp, wpage.data(), M * 4);
  std::memcpy(h + o_wo, woff.data(), M * 4);
  std::memcpy(h + o_rb, rowbt.data(), M * 4);
  if (!drows.empty()) std::memcpy(h + o_dr, drows.data(), drows.size() * 4);
  if (!tiles.empty()) std::memcpy(h + o_ti, tiles.data(), tiles.size() * 4);
  int* bt = h + o_bt;
  for (int s = 0; s < n_seqs_; ++s) {
    const auto& pg = cache_.pages(seqs[s]);
    int* row = bt + (size_t)s * width;
    std::copy(pg.begin(), pg.end(), row);
    std::fill(row + pg.size(), row + width, 0);
  }
  if (src) std::memcpy(h + o_src, src, M * 4);
  // No copy command: the step's embed launch reads its own inputs from the
  // host block and stages the whole block into d_meta for the launches after
  // it.  The other buffers' block may still be in use by the step queued
  // before; this one's last reader was the step two back, already waited for.
  const int* hd = (const int*)sb.hd_meta;
  hd_tok_ = hd + o_tok; hd_pos_ = hd + o_pos; hd_src_ = src ? hd + o_src : nullptr;
  int* d = (int*)sb.d_meta;
  d_pos_ = d + o_pos; d_wpage_ = d + o_wp; d_woff_ = d + o_wo; d_rowbt_ = d + o_rb;
  d_drows_ = d + o_dr; d_tiles_ = d + o_ti; d_bt_ = d + o_bt;
  stage_src_ = sb.hd_meta;
  stage_dst_ = sb.d_meta;
  meta_bytes_ = bytes;
  sb.M = M;
}

std::vector<int> TransformerRunner::signature() const {
  return {M_, n_decode_, n_tiles_, n_seqs_, bt_width_, max_kv_, split_tokens_, fused_proj_};
}

void TransformerRunner::enqueue_forward(int b, bool greedy, bool from_prev) {
  const int M = M_, D = cfg_.d_model, F = cfg_.mlp, V = cfg_.vocab;
  const int act = cfg_.act_dtype(), wd = cfg_.weight_dtype;
  hipStream_t s = stream_;
  int* const d_next = bufs_[b].d_next;
  // Rows with a token source read the previous step's greedy tokens (the
  // other buffers' results, which that step wrote earlier on this stream).
  cbis_check(cbis_embed_from(M, D, hd_tok_, from_prev ? hd_src_ : nullptr, from_prev ? bufs_[b ^ 1].d_next : nullptr,
                             hd_pos_, w_.emb_dtype(), w_.tok_emb, w_.pos_emb, V, cfg_.max_seq, d_x_, stage_src_,
                             stage_dst_, meta_bytes_, s),
             "embed + metadata staging");

  cbis_gemm_desc g = {};
  g.M = M;
  g.x_dtype = act;
  g.w_dtype = wd;

  cbis_attn_desc a = {};
  a.n_heads = cfg_.n_heads;
  a.head_dim = cfg_.head_dim;
  a.page_size = cfg_.page_size;
  a.q_dtype = CBIS_F32;
  a.q = d_q_;
  a.ldq = D;
  a.kv_dtype = cfg_.kv_dtype;
  a.num_pages = cache_.max_pages();
  a.block_table = d_bt_;
  a.bt_stride = bt_width_;
  a.row_bt = d_rowbt_;
  a.row_pos = d_pos_;
  a.out_dtype = act;
  a.out = d_attn_;
  a.ldo = D;
  a.max_kv_len = max_kv_;
  a.split_tokens = split_tokens_;
  a.workspace = d_ws_;
  a.workspace_bytes = ws_bytes_;
  a.tile_pages = 8;

  // LayerNorms that follow a residual GEMM (ln2 after the out-projection,
  // the next layer's ln1 or ln_f after fc2) run with it (cbis_gemm_layernorm:
  // fused with the GEMM's split-K reduce, where it splits).  Decode-sized
  // steps with short rows instead hand ln1 and ln2 to the QKV and fc1 GEMMs
  // that read them (cbis_layernorm_gemm forms them inside the skinny GEMM
  // for M <= 64 and rows of at most 512: two launches fewer per layer);
  // longer decode rows (config 5, d 2048) keep the fused reduce + LayerNorm,
  // which lets their out-projection and fc2 split K.
  const bool ln_pro = M <= 64 && D <= 512;
  if (!ln_pro)
    cbis_check(cbis_layernorm(M, D, d_x_, D, w_.layers[0].ln1_w, w_.layers[0].ln1_b, 1e-5f, act, d_xn_, D, s),
               "ln1");
  for (int l = 0; l < cfg_.n_layers; ++l) {
    const LayerWeights& L = w_.layers[l];
    // QKV projection; K and V columns go straight to their page slots.
    g = cbis_gemm_desc{};
    g.workspace = d_gemm_ws_; g.workspace_bytes = gemm_ws_bytes_;
    g.M = M; g.N = 3 * D; g.K = D;
    g.x_dtype = act; g.X = d_xn_; g.ldx = D;
    g.w_dtype = wd; g.W = L.wqkv; g.ldw = D; g.w_scale = L.sqkv;
    g.bias = L.bqkv;
    g.y_dtype = CBIS_F32; g.Y = d_q_; g.ldy = D;
    g.kv_col0 = D; g.kv_width = D; g.kv_dtype = cfg_.kv_dtype; g.page_size = cfg_.page_size;
    g.k_pool = cache_.k_base(l); g.v_pool = cache_.v_base(l);
    g.write_page = d_wpage_; g.write_offset = d_woff_;
    if (ln_pro) cbis_check(cbis_layernorm_gemm(&g, d_x_, D, L.ln1_w, L.ln1_b, 1e-5f, s), "ln1 + qkv gemm");
    else cbis_check(cbis_gemm(&g, s), "qkv gemm");
    a.k_pool = cache_.k_base(l);
    a.v_pool = cache_.v_base(l);
    a.n_rows = n_decode_;
    a.rows = d_drows_;
    // out-projection + bias + residual, in place on x
    g = cbis_gemm_desc{};
    g.workspace = d_gemm_ws_; g.workspace_bytes = gemm_ws_bytes_;
    g.M = M; g.N = D; g.K = D;
    g.x_dtype = act; g.X = d_attn_; g.ldx = D;
    g.w_dtype = wd; g.W = L.wo; g.ldw = D; g.w_scale = L.so;
    g.bias = L.bo; g.residual = d_x_; g.ldr = D;
    g.y_dtype = CBIS_F32; g.Y = d_x_; g.ldy = D;
    if (fused_proj_) {
      cbis_check(cbis_paged_attention_proj(&a, &g, s), "attention + out-proj");
    } else {
      // Single rows on the split-KV decode kernel, runs of rows on the MFMA
      // prefill kernel (whose launch also merges the decode rows' splits).
      cbis_check(cbis_paged_attention_mixed(&a, n_tiles_, d_tiles_, s), "attention");
      if (ln_pro) cbis_check(cbis_gemm(&g, s), "out-proj gemm");
      else cbis_check(cbis_gemm_layernorm(&g, L.ln2_w, L.ln2_b, 1e-5f, act, d_xn_, D, s), "out-proj gemm + ln2");
    }
    g = cbis_gemm_desc{};
    g.workspace = d_gemm_ws_; g.workspace_bytes = gemm_ws_bytes_;
    g.M = M; g.N = F; g.K = D;
    g.x_dtype = act; g.X = d_xn_; g.ldx = D;
    g.w_dtype = wd; g.W = L.w1; g.ldw = D; g.w_scale = L.s1;
    g.bias = L.b1; g.epilogue = CBIS_EPI_GELU;
    g.y_dtype = act; g.Y = d_h_; g.ldy = F;
    if (ln_pro) cbis_check(cbis_layernorm_gemm(&g, d_x_, D, L.ln2_w, L.ln2_b, 1e-5f, s), "ln2 + fc1 gemm");
    else cbis_check(cbis_gemm(&g, s), "fc1 gemm");
    g = cbis_gemm_desc{};
    g.workspace = d_gemm_ws_; g.workspace_bytes = gemm_ws_bytes_;
    g.M = M; g.N = D; g.K = F;
    g.x_dtype = act; g.X = d_h_; g.ldx = F;
    g.w_dtype = wd; g.W = L.w2; g.ldw = F; g.w_scale = L.s2;
    g.bias = L.b2; g.residual = d_x_; g.ldr = D;
    g.y_dtype = CBIS_F32; g.Y = d_x_; g.ldy = D;
    const bool last = l + 1 == cfg_.n_layers;
    const float* nw = last ? w_.ln_f_w : w_.layers[l + 1].ln1_w;
    const float* nb = last ? w_.ln_f_b : w_.layers[l + 1].ln1_b;
    if (ln_pro) cbis_check(cbis_gemm(&g, s), "fc2 gemm");
    else
      cbis_check(cbis_gemm_layernorm(&g, nw, nb, 1e-5f, act, d_xn_, D, s), last ? "fc2 gemm + ln_f" : "fc2 gemm + ln1");
  }
  g = cbis_gemm_desc{};
  g.workspace = d_gemm_ws_; g.workspace_bytes = gemm_ws_bytes_;
  g.M = M; g.N = V; g.K = D;
  g.x_dtype = act; g.X = d_xn_; g.ldx = D;
  g.w_dtype = wd; g.W = w_.lm_head; g.ldw = D; g.w_scale = w_.lm_scale;
  g.y_dtype = CBIS_F32; g.Y = d_logits_; g.ldy = V;
  float* margins = (float*)(d_next + M);
  if (ln_pro && greedy)
    cbis_check(cbis_layernorm_gemm_argmax(&g, d_x_, D, w_.ln_f_w, w_.ln_f_b, 1e-5f, d_next, margins, d_amax_ws_,
                                          amax_ws_bytes_, s),
               "ln_f + lm_head gemm + argmax");
  else if (ln_pro)
    cbis_check(cbis_layernorm_gemm(&g, d_x_, D, w_.ln_f_w, w_.ln_f_b, 1e-5f, s), "ln_f + lm_head gemm");
  else if (greedy)
    cbis_check(cbis_gemm_argmax(&g, d_next, margins, d_amax_ws_, amax_ws_bytes_, s), "lm_head gemm + argmax");
  else
    cbis_check(cbis_gemm(&g, s), "lm_head gemm");
}

void TransformerRunner::run_step(int b, bool greedy, bool from_prev) {
  auto body = [&]() { enqueue_forward(b, greedy, from_prev); };
  if (!use_graphs_) {
    body();
    return;
  }
  // A graph names one set of step buffers (and, reading the previous step's
  // tokens, the other set's results).
  std::vector<int> sig = signature();
  sig.insert(sig.end(), {greedy ? 1 : 0, b, from_prev ? 1 : 0});
  auto it = graphs_.find(sig);
  if (it == graphs_.end()) {
    if (graphs_.size() >= kMaxGraphs) {
      hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");  // a queued step may run one of them
      for (auto& g : graphs_) (void)hipGraphExecDestroy(g.second.exec);
      graphs_.clear();
    }
    hipGraph_t graph = nullptr;
    hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
      body();
    } catch (...) {
      (void)hipStreamEndCapture(stream_, &graph);
      if (graph) (void)hipGraphDestroy(graph);
      throw;
    }
    hip_check(hipStreamEndCapture(stream_, &graph), "hipStreamEndCapture");
    GraphEntry e;
    hipError_t rc = hipGraphInstantiate(&e.exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    hip_check(rc, "hipGraphInstantiate");
    it = graphs_.emplace(sig, e).first;
  }
  hip_check(hipGraphLaunch(it->second.exec, stream_), "hipGraphLaunch");
}

void TransformerRunner::timed_step(int b, bool greedy, bool from_prev) {
  hip_check(hipEventRecord(bufs_[b].ev_start, stream_), "hipEventRecord");
  run_step(b, greedy, from_prev);
  hip_check(hipEventRecord(bufs_[b].ev_stop, stream_), "hipEventRecord");
}

std::vector<float> TransformerRunner::forward_step(const std::vector<int>& token_ids, const std::vector<int>& positions,
                                                   const std::vector<int>& seq_ids) {
  margins_.clear();
  const int M = (int)token_ids.size();
  if (M == 0) return {};
  if ((int)positions.size() != M || (int)seq_ids.size() != M)
    throw std::invalid_argument("forward_step: token_ids/positions/seq_ids sizes differ");
  const int b = next_buf_;
  if (bufs_[b].pending) throw std::logic_error("forward_step: a queued greedy step has not been waited for");
  prepare(b, token_ids.data(), positions.data(), seq_ids.data(), nullptr, M);
  timed_step(b, false, false);
  std::vector<float> logits((size_t)M * cfg_.vocab);
  hip_check(hipMemcpyAsync(logits.data(), d_logits_, logits.size() * 4, hipMemcpyDeviceToHost, stream_), "D2H logits");
  hip_check(hipStreamSynchronize(stream_), "forward_step sync");
  hip_check(hipEventElapsedTime(&last_device_ms_, bufs_[b].ev_start, bufs_[b].ev_stop), "hipEventElapsedTime");
  bufs_[b].ticket = -1;
  next_buf_ ^= 1;
  prev_greedy_rows_ = -1;  // no greedy tokens for the next step to read
  return logits;
}

int64_t TransformerRunner::enqueue_greedy(const std::vector<int>& token_ids, const std::vector<int>& positions,
                                          const std::vector<int>& seq_ids, const std::vector<int>& token_src) {
  const int M = (int)token_ids.size();
  if (M == 0) throw std::invalid_argument("enqueue_greedy: no rows");
  if ((int)positions.size() != M || (int)seq_ids.size() != M)
    throw std::invalid_argument("enqueue_greedy: token_ids/positions/seq_ids sizes differ");
  if (!token_src.empty() && (int)token_src.size() != M)
    throw std::invalid_argument("enqueue_greedy: token_src must be empty or have one entry per row");
  const int b = next_buf_;
  StepBuf& sb = bufs_[b];
  if (sb.pending) throw std::logic_error("enqueue_greedy: the step two before this one has not been waited for");
  bool from_prev = false;
  for (int v : token_src) from_prev = from_prev || v >= 0;
  if (from_prev && prev_greedy_rows_ < 0)
    throw std::logic_error("enqueue_greedy: token_src needs a greedy step enqueued just before");
  using clk = std::chrono::steady_clock;
  const auto t0 = clk::now();
  prepare(b, token_ids.data(), positions.data(), seq_ids.data(), from_prev ? token_src.data() : nullptr, M);
  const auto t1 = clk::now();
  timed_step(b, true, from_prev);  // its argmax stores tokens and margins in sb.h_next
  const auto t2 = clk::now();
  auto ms = [](clk::duration d) { return std::chrono::duration<double, std::milli>(d).count(); };
  sb.host_ms[0] = ms(t1 - t0);
  sb.host_ms[1] = ms(t2 - t1);
  sb.pending = true;
  sb.ticket = tickets_++;
  next_buf_ ^= 1;
  prev_greedy_rows_ = M;
  return sb.ticket;
}

std::vector<int> TransformerRunner::wait_greedy(int64_t ticket) {
  int b = -1;
  for (int i = 0; i < 2; ++i)
    if (bufs_[i].pending && bufs_[i].ticket == ticket) b = i;
  if (b < 0) throw std::invalid_argument("wait_greedy: no queued greedy step has this ticket");
  StepBuf& sb = bufs_[b];
  using clk = std::chrono::steady_clock;
  const auto t0 = clk::now();
  hip_check(hipEventSynchronize(sb.ev_stop), "wait_greedy sync");
  const auto t1 = clk::now();
  sb.pending = false;
  hip_check(hipEventElapsedTime(&last_device_ms_, sb.ev_start, sb.ev_stop), "hipEventElapsedTime");
  host_ms_[0] = sb.host_ms[0];
  host_ms_[1] = sb.host_ms[1];
  host_ms_[2] = std::chrono::duration<double, std::milli>(t1 - t0).count();
  const int M = sb.M;
  margins_.assign((const float*)(sb.h_next + M), (const float*)(sb.h_next + M) + M);
  return std::vector<int>(sb.h_next, sb.h_next + M);
}

std::vector<int> TransformerRunner::forward_step_greedy(const std::vector<int>& token_ids,
                                                        const std::vector<int>& positions,
                                                        const std::vector<int>& seq_ids) {
  margins_.clear();
  if (token_ids.empty()) return {};
  return wait_greedy(enqueue_greedy(token_ids, positions, seq_ids, {}));
}

}  // namespace cbis
