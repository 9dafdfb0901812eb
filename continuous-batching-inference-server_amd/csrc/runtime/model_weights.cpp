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

}  // namespace

// Tensor table of the device arena, in a fixed order; every tensor starts on a
// 256-byte boundary.
std::vector<ModelWeights::Entry> ModelWeights::layout(const ModelConfig& cfg) {
  cfg.validate();
  const size_t D = cfg.d_model, F = cfg.mlp, V = cfg.vocab, S = cfg.max_seq;
  const int wd = cfg.weight_dtype, ed = cfg.weight_dtype == CBIS_F32 ? CBIS_F32 : CBIS_BF16;
  const size_t we = dtype_size(wd), ee = dtype_size(ed);
  const bool fp8 = wd == CBIS_FP8E4M3;
  std::vector<Entry> t;
  size_t off = 0;
  auto add = [&](const std::string& name, int dtype, size_t bytes) {
    t.push_back({name, dtype, off, bytes});
    off = align256(off + bytes);
  };
  add("tok_emb", ed, V * D * ee);
  add("pos_emb", ed, S * D * ee);
  for (int l = 0; l < cfg.n_layers; ++l) {
    const std::string pre = "l" + std::to_string(l) + ".";
    add(pre + "ln1_w", CBIS_F32, D * 4); add(pre + "ln1_b", CBIS_F32, D * 4);
    add(pre + "ln2_w", CBIS_F32, D * 4); add(pre + "ln2_b", CBIS_F32, D * 4);
    add(pre + "wqkv", wd, 3 * D * D * we); add(pre + "bqkv", CBIS_F32, 3 * D * 4);
    add(pre + "wo", wd, D * D * we); add(pre + "bo", CBIS_F32, D * 4);
    add(pre + "w1", wd, F * D * we); add(pre + "b1", CBIS_F32, F * 4);
    add(pre + "w2", wd, D * F * we); add(pre + "b2", CBIS_F32, D * 4);
    if (fp8) {
      add(pre + "sqkv", CBIS_F32, 3 * D * 4); add(pre + "so", CBIS_F32, D * 4);
      add(pre + "s1", CBIS_F32, F * 4); add(pre + "s2", CBIS_F32, D * 4);
    }
  }
  add("ln_f_w", CBIS_F32, D * 4);
  add("ln_f_b", CBIS_F32, D * 4);
  add("lm_head", wd, V * D * we);
  if (fp8) add("lm_scale", CBIS_F32, V * 4);
  return t;
}

namespace {
}  // namespace

ModelWeights::~ModelWeights() { free_all(); }

void ModelWeights::free_all() {
  if (arena_) (void)hipFree(arena_);
  arena_ = nullptr;
  arena_bytes_ = 0;
}

void ModelWeights::plan() {
  table_ = layout(cfg);
  arena_bytes_ = table_.back().offset + table_.back().bytes;
  hip_check(hipMalloc((void**)&arena_, arena_bytes_), "ModelWeights: hipMalloc");
  named_.clear();
  for (const auto& e : table_) named_[e.name] = arena_ + e.offset;
  auto f32 = [&](const std::string& n) { return (float*)named_.at(n); };
  tok_emb = named_.at("tok_emb");
  pos_emb = named_.at("pos_emb");
  layers.assign(cfg.n_layers, LayerWeights());
  const bool fp8 = cfg.weight_dtype == CBIS_FP8E4M3;
  for (int l = 0; l < cfg.n_layers; ++l) {
    LayerWeights& L = layers[l];
    const std::string pre = "l" + std::to_string(l) + ".";
    L.ln1_w = f32(pre + "ln1_w"); L.ln1_b = f32(pre + "ln1_b");
    L.ln2_w = f32(pre + "ln2_w"); L.ln2_b = f32(pre + "ln2_b");
    L.wqkv = named_.at(pre + "wqkv"); L.bqkv = f32(pre + "bqkv");
    L.wo = named_.at(pre + "wo"); L.bo = f32(pre + "bo");
    L.w1 = named_.at(pre + "w1"); L.b1 = f32(pre + "b1");
    L.w2 = named_.at(pre + "w2"); L.b2 = f32(pre + "b2");
    if (fp8) { L.sqkv = f32(pre + "sqkv"); L.so = f32(pre + "so"); L.s1 = f32(pre + "s1"); L.s2 = f32(pre + "s2"); }
  }
  ln_f_w = f32("ln_f_w");
  ln_f_b = f32("ln_f_b");
  lm_head = named_.at("lm_head");
  lm_scale = fp8 ? f32("lm_scale") : nullptr;
  // names the C-ABI has always resolved, null for a model without fp8 scales
  for (int l = 0; l < cfg.n_layers && !fp8; ++l)
    for (const char* n : {"sqkv", "so", "s1", "s2"}) named_["l" + std::to_string(l) + "." + n] = nullptr;
  if (!fp8) named_["lm_scale"] = nullptr;
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
  cfg.validate();
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw std::runtime_error("cannot open " + path);
  const size_t nbytes = (size_t)f.tellg();
  // The file is the config's fp32 tensors back to back, nothing else
  // (python/export_weights.py:42-66): a size that differs means other dims.
  {
    const size_t D = cfg.d_model, F = cfg.mlp, V = cfg.vocab, S = cfg.max_seq;
    const size_t per_layer = 2 * D + 4 * (D * D + D) + 2 * D + F * D + F + D * F + D;
    const size_t want = (V * D + S * D + cfg.n_layers * per_layer + 2 * D + V * D) * 4;
    if (nbytes != want)
      throw std::runtime_error("weights.bin: " + std::to_string(nbytes) + " bytes, the config's tensors are " +
                               std::to_string(want) + " bytes");
  }
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

// ---------------------------------------------------------------------------
// Packed checkpoint format (little-endian), version 1:
//   char[8]  magic "CBISWT01"
//   u32      version (1), u32 tensor count
//   i32[10]  vocab, d_model, n_heads, head_dim, n_layers, mlp, max_seq,
//            page_size, weight_dtype, kv_dtype
//   u64      arena bytes, u64 data offset (4096-aligned), u64 checksum
//   per tensor: u16 name length, name, u32 dtype, u64 offset, u64 bytes
//   zero padding to the data offset, then the arena image.
// The checksum folds the image as 64-bit words: h = rotl(h, 5) ^ w, times an
// odd constant.  A loader rejects a file whose table differs from the layout
// its config implies, whose size falls short, or whose checksum differs.
// ---------------------------------------------------------------------------
namespace {
constexpr char kMagic[8] = {'C', 'B', 'I', 'S', 'W', 'T', '0', '1'};
constexpr uint32_t kVersion = 1;

uint64_t fold(uint64_t h, const uint8_t* p, size_t n) {
  size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    uint64_t w;
    std::memcpy(&w, p + i, 8);
    h = ((h << 5) | (h >> 59)) ^ w;
    h *= 0x9E3779B97F4A7C15ULL;
  }
  for (; i < n; ++i) {
    h = ((h << 5) | (h >> 59)) ^ p[i];
    h *= 0x9E3779B97F4A7C15ULL;
  }
  return h;
}

template <typename T>
void put(std::vector<uint8_t>& b, T v) {
  const size_t o = b.size();
  b.resize(o + sizeof(T));
  std::memcpy(b.data() + o, &v, sizeof(T));
}

struct Reader {
  const std::vector<uint8_t>& b;
  size_t o = 0;
  template <typename T>
  T get() {
    if (o + sizeof(T) > b.size()) throw std::runtime_error("packed weights: header truncated");
    T v;
    std::memcpy(&v, b.data() + o, sizeof(T));
    o += sizeof(T);
    return v;
  }
};

// 4 MiB pinned bounce buffer for the host <-> device image copies.
struct Bounce {
  uint8_t* p = nullptr;
  static constexpr size_t kBytes = (size_t)4 << 20;
  Bounce() { hip_check(hipHostMalloc((void**)&p, kBytes, 0), "packed weights: hipHostMalloc"); }
  ~Bounce() { (void)hipHostFree(p); }
};
}  // namespace

void ModelWeights::save_packed(const std::string& path) const {
  std::vector<uint8_t> hdr(kMagic, kMagic + 8);
  put<uint32_t>(hdr, kVersion);
  put<uint32_t>(hdr, (uint32_t)table_.size());
  for (int v : {cfg.vocab, cfg.d_model, cfg.n_heads, cfg.head_dim, cfg.n_layers, cfg.mlp, cfg.max_seq, cfg.page_size,
                cfg.weight_dtype, cfg.kv_dtype})
    put<int32_t>(hdr, v);
  const size_t fixed = hdr.size();
  put<uint64_t>(hdr, arena_bytes_);
  put<uint64_t>(hdr, 0);  // data offset, patched below
  put<uint64_t>(hdr, 0);  // checksum, patched below
  for (const auto& e : table_) {
    put<uint16_t>(hdr, (uint16_t)e.name.size());
    hdr.insert(hdr.end(), e.name.begin(), e.name.end());
    put<uint32_t>(hdr, (uint32_t)e.dtype);
    put<uint64_t>(hdr, (uint64_t)e.offset);
    put<uint64_t>(hdr, (uint64_t)e.bytes);
  }
  const uint64_t data_off = (hdr.size() + 4095) & ~(uint64_t)4095;
  std::memcpy(hdr.data() + fixed + 8, &data_off, 8);

  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) throw std::runtime_error("cannot create " + path);
  std::vector<uint8_t> pad(data_off - hdr.size(), 0);
  f.write((const char*)hdr.data(), (std::streamsize)hdr.size());
  f.write((const char*)pad.data(), (std::streamsize)pad.size());
  Bounce bb;
  uint64_t h = 0;
  for (size_t o = 0; o < arena_bytes_; o += Bounce::kBytes) {
    const size_t n = std::min(Bounce::kBytes, arena_bytes_ - o);
    hip_check(hipMemcpy(bb.p, arena_ + o, n, hipMemcpyDeviceToHost), "packed weights: D2H");
    h = fold(h, bb.p, n);
    f.write((const char*)bb.p, (std::streamsize)n);
  }
  f.seekp((std::streamoff)(fixed + 16));
  f.write((const char*)&h, 8);
  if (!f) throw std::runtime_error("write failed: " + path);
}

std::unique_ptr<ModelWeights> ModelWeights::load_packed(const std::string& path) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw std::runtime_error("cannot open " + path);
  const uint64_t fsize = (uint64_t)f.tellg();
  f.seekg(0);
  std::vector<uint8_t> head(std::min<uint64_t>(fsize, 1 << 20));
  f.read((char*)head.data(), (std::streamsize)head.size());
  Reader r{head};
  char magic[8];
  for (char& c : magic) c = r.get<char>();
  if (std::memcmp(magic, kMagic, 8) != 0) throw std::runtime_error("packed weights: bad magic in " + path);
  const uint32_t version = r.get<uint32_t>();
  if (version != kVersion) throw std::runtime_error("packed weights: unsupported version " + std::to_string(version));
  const uint32_t count = r.get<uint32_t>();
  ModelConfig cfg;
  int* fields[10] = {&cfg.vocab, &cfg.d_model, &cfg.n_heads, &cfg.head_dim, &cfg.n_layers,
                     &cfg.mlp, &cfg.max_seq, &cfg.page_size, &cfg.weight_dtype, &cfg.kv_dtype};
  for (int* p : fields) *p = r.get<int32_t>();
  const uint64_t arena = r.get<uint64_t>(), data_off = r.get<uint64_t>(), sum = r.get<uint64_t>();
  const std::vector<Entry> want = layout(cfg);  // validates the config
  if (count != want.size()) throw std::runtime_error("packed weights: tensor count does not match the config");
  for (const auto& e : want) {
    const uint16_t len = r.get<uint16_t>();
    std::string name(len, '\0');
    for (char& c : name) c = r.get<char>();
    const uint32_t dtype = r.get<uint32_t>();
    const uint64_t off = r.get<uint64_t>(), bytes = r.get<uint64_t>();
    if (name != e.name || (int)dtype != e.dtype || off != e.offset || bytes != e.bytes)
      throw std::runtime_error("packed weights: tensor table differs from the layout at " + e.name);
  }
  if (arena != want.back().offset + want.back().bytes) throw std::runtime_error("packed weights: arena size differs");
  if (data_off < r.o || data_off % 4096 || data_off + arena > fsize)
    throw std::runtime_error("packed weights: file truncated or data offset invalid");

  std::unique_ptr<ModelWeights> w(new ModelWeights());
  w->cfg = cfg;
  w->plan();
  f.seekg((std::streamoff)data_off);
  Bounce bb;
  uint64_t h = 0;
  for (size_t o = 0; o < arena; o += Bounce::kBytes) {
    const size_t n = std::min<size_t>(Bounce::kBytes, arena - o);
    f.read((char*)bb.p, (std::streamsize)n);
    if (!f) throw std::runtime_error("packed weights: read failed");
    h = fold(h, bb.p, n);
    hip_check(hipMemcpy(w->arena_ + o, bb.p, n, hipMemcpyHostToDevice), "packed weights: H2D");
  }
  if (h != sum) throw std::runtime_error("packed weights: checksum mismatch");
  return w;
}

}  // namespace cbis
