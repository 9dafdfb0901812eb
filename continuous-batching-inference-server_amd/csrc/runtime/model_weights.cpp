// ModelWeights: the reference's weights.bin loader (src/model_weights.cpp:41-75,
// order python/export_weights.py:42-66) plus the seeded synthetic init the
// benchmark configurations use.  Every tensor lives in one device arena;
// linear weights are stored in the config's dtype, with Q/K/V fused into one
// [3d, d] matrix so the QKV projection is a single GEMM.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>

#include "runtime.hpp"

namespace cbis {

namespace {

// Synthetic-weight stream ids (one counter-based N(0, std) stream per tensor,
// element index = row-major offset).  Q/K/V rows come from their own streams
// and are concatenated into the fused matrix.
constexpr uint64_t kStreamTokEmb = 1, kStreamPosEmb = 2, kStreamLmHead = 3;
constexpr uint64_t kLayerBase = 100, kLayerStride = 20;
enum LayerTensor { kWq, kBq, kWk, kBk, kWv, kBv, kWo, kBo, kFc1, kB1, kFc2, kB2 };
uint64_t layer_stream(int l, LayerTensor t) { return kLayerBase + kLayerStride * (uint64_t)l + (uint64_t)t; }

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Lays tensors out in the arena in a fixed order.
struct Planner {
  size_t off = 0;
  std::vector<std::pair<void**, size_t>> slots;
  template <typename T>
  void add(T** p, size_t bytes) {
    slots.push_back({(void**)p, off});
    off = align256(off + bytes);
  }
};

}  // namespace

ModelWeights::~ModelWeights() { free_all(); }

void ModelWeights::free_all() {
  if (arena_) (void)hipFree(arena_);
  arena_ = nullptr;
  arena_bytes_ = 0;
}

void ModelWeights::plan() {
  cfg.validate();
  const size_t D = cfg.d_model, F = cfg.mlp, V = cfg.vocab, S = cfg.max_seq;
  const size_t we = dtype_size(cfg.weight_dtype), ee = dtype_size(emb_dtype());
  const bool fp8 = cfg.weight_dtype == CBIS_FP8E4M3;
  Planner p;
  p.add(&tok_emb, V * D * ee);
  p.add(&pos_emb, S * D * ee);
  layers.assign(cfg.n_layers, LayerWeights());
  for (auto& L : layers) {
    p.add(&L.ln1_w, D * 4); p.add(&L.ln1_b, D * 4);
    p.add(&L.ln2_w, D * 4); p.add(&L.ln2_b, D * 4);
    p.add(&L.wqkv, 3 * D * D * we); p.add(&L.bqkv, 3 * D * 4);
    p.add(&L.wo, D * D * we); p.add(&L.bo, D * 4);
    p.add(&L.w1, F * D * we); p.add(&L.b1, F * 4);
    p.add(&L.w2, D * F * we); p.add(&L.b2, D * 4);
    if (fp8) { p.add(&L.sqkv, 3 * D * 4); p.add(&L.so, D * 4); p.add(&L.s1, F * 4); p.add(&L.s2, D * 4); }
  }
  p.add(&ln_f_w, D * 4);
  p.add(&ln_f_b, D * 4);
  p.add(&lm_head, V * D * we);
  if (fp8) p.add(&lm_scale, V * 4);
  hip_check(hipMalloc((void**)&arena_, p.off), "ModelWeights: hipMalloc");
  arena_bytes_ = p.off;
  for (auto& s : p.slots) *s.first = arena_ + s.second;

  named_.clear();
  named_["tok_emb"] = tok_emb; named_["pos_emb"] = pos_emb; named_["lm_head"] = lm_head;
  named_["lm_scale"] = lm_scale; named_["ln_f_w"] = ln_f_w; named_["ln_f_b"] = ln_f_b;
  for (int l = 0; l < cfg.n_layers; ++l) {
    const auto& L = layers[l];
    const std::string pre = "l" + std::to_string(l) + ".";
    named_[pre + "wqkv"] = L.wqkv; named_[pre + "bqkv"] = L.bqkv; named_[pre + "sqkv"] = L.sqkv;
    named_[pre + "wo"] = L.wo; named_[pre + "bo"] = L.bo; named_[pre + "so"] = L.so;
    named_[pre + "w1"] = L.w1; named_[pre + "b1"] = L.b1; named_[pre + "s1"] = L.s1;
    named_[pre + "w2"] = L.w2; named_[pre + "b2"] = L.b2; named_[pre + "s2"] = L.s2;
    named_[pre + "ln1_w"] = L.ln1_w; named_[pre + "ln1_b"] = L.ln1_b;
    named_[pre + "ln2_w"] = L.ln2_w; named_[pre + "ln2_b"] = L.ln2_b;
  }
}

void* ModelWeights::tensor(const std::string& name) const {
  auto it = named_.find(name);
  if (it == named_.end()) throw std::out_of_range("ModelWeights: no tensor " + name);
  return it->second;
}

namespace {

// Converts an fp32 device staging buffer into a weight slot of `dtype`
// (fp8: per-row quantisation into codes + scale).
void store_linear(const float* src, int rows, int cols, int dtype, void* dst, float* scale, hipStream_t s) {
  if (dtype == CBIS_FP8E4M3)
    cbis_check(cbis_quantize_fp8_rows((uint8_t*)dst, scale, src, rows, cols, s), "quantize fp8");
  else
    cbis_check(cbis_convert_f32(dst, dtype, src, (int64_t)rows * cols, s), "convert weights");
}

void fill_const(float* dst, size_t n, float v, hipStream_t s) {
  std::vector<float> h(n, v);
  hip_check(hipMemcpyAsync(dst, h.data(), n * 4, hipMemcpyHostToDevice, s), "fill_const");
  hip_check(hipStreamSynchronize(s), "fill_const sync");
}

}  // namespace

std::unique_ptr<ModelWeights> ModelWeights::synthetic(const ModelConfig& cfg, uint64_t seed, float std) {
  std::unique_ptr<ModelWeights> w(new ModelWeights());
  w->cfg = cfg;
  w->plan();
  const int D = cfg.d_model, F = cfg.mlp, V = cfg.vocab, S = cfg.max_seq;
  const int wd = cfg.weight_dtype, ed = w->emb_dtype();
  hipStream_t s = nullptr;
  // fp32 staging for one linear weight at a time (largest: lm_head / fc).
  const size_t stage_elems = std::max<size_t>({(size_t)V * D, (size_t)F * D, (size_t)3 * D * D});
  float* stage = nullptr;
  hip_check(hipMalloc((void**)&stage, stage_elems * 4), "ModelWeights: staging");
  auto gen = [&](void* dst, int dtype, int64_t n, uint64_t stream_id) {
    cbis_check(cbis_fill_normal_exact(dst, dtype, n, seed, stream_id, 0, std, s), "fill_normal_exact");
  };
  try {
    gen(w->tok_emb, ed, (int64_t)V * D, kStreamTokEmb);
    gen(w->pos_emb, ed, (int64_t)S * D, kStreamPosEmb);
    for (int l = 0; l < cfg.n_layers; ++l) {
      LayerWeights& L = w->layers[l];
      const int64_t dd = (int64_t)D * D;
      gen(stage, CBIS_F32, dd, layer_stream(l, kWq));
      gen(stage + dd, CBIS_F32, dd, layer_stream(l, kWk));
      gen(stage + 2 * dd, CBIS_F32, dd, layer_stream(l, kWv));
      store_linear(stage, 3 * D, D, wd, L.wqkv, L.sqkv, s);
      gen(L.bqkv, CBIS_F32, D, layer_stream(l, kBq));
      gen(L.bqkv + D, CBIS_F32, D, layer_stream(l, kBk));
      gen(L.bqkv + 2 * D, CBIS_F32, D, layer_stream(l, kBv));
      hip_check(hipStreamSynchronize(s), "sync");
      gen(stage, CBIS_F32, dd, layer_stream(l, kWo));
      store_linear(stage, D, D, wd, L.wo, L.so, s);
      gen(L.bo, CBIS_F32, D, layer_stream(l, kBo));
      hip_check(hipStreamSynchronize(s), "sync");
      gen(stage, CBIS_F32, (int64_t)F * D, layer_stream(l, kFc1));
      store_linear(stage, F, D, wd, L.w1, L.s1, s);
      gen(L.b1, CBIS_F32, F, layer_stream(l, kB1));
      hip_check(hipStreamSynchronize(s), "sync");
      gen(stage, CBIS_F32, (int64_t)D * F, layer_stream(l, kFc2));
      store_linear(stage, D, F, wd, L.w2, L.s2, s);
      gen(L.b2, CBIS_F32, D, layer_stream(l, kB2));
      hip_check(hipStreamSynchronize(s), "sync");
      fill_const(L.ln1_w, D, 1.f, s); fill_const(L.ln1_b, D, 0.f, s);
      fill_const(L.ln2_w, D, 1.f, s); fill_const(L.ln2_b, D, 0.f, s);
    }
    fill_const(w->ln_f_w, D, 1.f, s);
    fill_const(w->ln_f_b, D, 0.f, s);
    gen(stage, CBIS_F32, (int64_t)V * D, kStreamLmHead);
    store_linear(stage, V, D, wd, w->lm_head, w->lm_scale, s);
    hip_check(hipStreamSynchronize(s), "ModelWeights::synthetic sync");
  } catch (...) {
    (void)hipFree(stage);
    throw;
  }
  hip_check(hipFree(stage), "ModelWeights: free staging");
  return w;
}

std::unique_ptr<ModelWeights> ModelWeights::load(const std::string& path, const ModelConfig& cfg) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw std::runtime_error("cannot open " + path);
  const size_t nbytes = (size_t)f.tellg();
  f.seekg(0);
  std::vector<float> buf(nbytes / 4);
  f.read(reinterpret_cast<char*>(buf.data()), (std::streamsize)(buf.size() * 4));
  size_t pos = 0;
  auto take = [&](size_t count) -> const float* {
    if (pos + count > buf.size()) throw std::runtime_error("weights.bin truncated");
    const float* p = buf.data() + pos;
    pos += count;
    return p;
  };

  std::unique_ptr<ModelWeights> w(new ModelWeights());
  w->cfg = cfg;
  w->plan();
  const size_t D = cfg.d_model, F = cfg.mlp, V = cfg.vocab, S = cfg.max_seq;
  const int wd = cfg.weight_dtype, ed = w->emb_dtype();
  hipStream_t s = nullptr;
  const size_t stage_elems = std::max<size_t>({V * D, S * D, F * D, 3 * D * D});
  float* stage = nullptr;
  hip_check(hipMalloc((void**)&stage, stage_elems * 4), "ModelWeights: staging");
  auto up = [&](float* dst, const float* src, size_t n) {
    hip_check(hipMemcpy(dst, src, n * 4, hipMemcpyHostToDevice), "ModelWeights: upload");
  };
  auto up_conv = [&](void* dst, int dtype, const float* src, size_t n) {
    up(stage, src, n);
    cbis_check(cbis_convert_f32(dst, dtype, stage, (int64_t)n, s), "convert");
    hip_check(hipStreamSynchronize(s), "sync");
  };
  auto up_linear = [&](void* dst, float* scale, const float* src, int rows, int cols) {
    up(stage, src, (size_t)rows * cols);
    store_linear(stage, rows, cols, wd, dst, scale, s);
    hip_check(hipStreamSynchronize(s), "sync");
  };
  try {
    up_conv(w->tok_emb, ed, take(V * D), V * D);
    up_conv(w->pos_emb, ed, take(S * D), S * D);
    std::vector<float> qkv(3 * D * D), bqkv(3 * D);
    for (auto& L : w->layers) {
      up(L.ln1_w, take(D), D);
      up(L.ln1_b, take(D), D);
      for (int j = 0; j < 3; ++j) {  // wq, bq, wk, bk, wv, bv
        std::memcpy(qkv.data() + j * D * D, take(D * D), D * D * 4);
        std::memcpy(bqkv.data() + j * D, take(D), D * 4);
      }
      up_linear(L.wqkv, L.sqkv, qkv.data(), 3 * (int)D, (int)D);
      up(L.bqkv, bqkv.data(), 3 * D);
      up_linear(L.wo, L.so, take(D * D), (int)D, (int)D);
      up(L.bo, take(D), D);
      up(L.ln2_w, take(D), D);
      up(L.ln2_b, take(D), D);
      up_linear(L.w1, L.s1, take(F * D), (int)F, (int)D);
      up(L.b1, take(F), F);
      up_linear(L.w2, L.s2, take(D * F), (int)D, (int)F);
      up(L.b2, take(D), D);
    }
    up(w->ln_f_w, take(D), D);
    up(w->ln_f_b, take(D), D);
    up_linear(w->lm_head, w->lm_scale, take(V * D), (int)V, (int)D);
  } catch (...) {
    (void)hipFree(stage);
    throw;
  }
  hip_check(hipFree(stage), "ModelWeights: free staging");
  return w;
}

}  // namespace cbis
