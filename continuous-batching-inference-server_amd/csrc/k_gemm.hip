// Flattened continuous-batch linear layers on gfx950 MFMA.
//
// Reference: linear_forward, kernels/linear.cu:15-34 -- cuBLAS SGEMM on the
// row-major Y[T,out] = X[T,in] . W[out,in]^T identity of docs/gemm_layout.md
// :16-41, then a separate bias launch (add_bias_rowmajor, :6-12), and in
// src/transformer.cpp:82-89 separate GELU and residual launches.  Here one
// kernel computes Y = epilogue(X . W^T) with the epilogue (per-channel fp8
// scale, bias, exact-erf GELU, fp32 residual, K/V page scatter) applied to
// the accumulators before the single store.
//
// Tiling.  Both operands are K-contiguous, so A (X) and B (W) tiles are
// staged the same way: rows of 128 bytes of K (64 bf16 / 32 fp32) in LDS,
// with the 16-byte chunk index XOR-swizzled by ((row >> 1) & 7) so the
// ds_read_b128 fragment loads of 16 consecutive rows hit distinct banks.
// Two LDS buffers; the next K tile is fetched into registers while the
// current one feeds the MFMAs (one barrier per K step).  Each wave owns a
// (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks:
//   bf16 / fp8:  v_mfma_f32_32x32x16_bf16 (fp8 weights are decoded to bf16
//                exactly when stored to LDS; the per-channel scale is applied
//                in the epilogue),
//   fp32:        v_mfma_f32_32x32x2_f32, four per ds_read_b128 fragment.
// Workgroups are renumbered so that each XCD (dispatch is round-robin over
// the 8 XCDs) receives a contiguous run of tiles, M-tile fastest, so the
// workgroups sharing a W column block share one L2.
// Optional split-K (gridDim.z) writes fp32 partials to a caller workspace
// and a second kernel reduces them and applies the epilogue.
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace cbis {
namespace {

struct GemmArgs {
  int M, N, K;
  const void* X;
  int64_t ldx;
  const void* W;
  int64_t ldw;
  const float* w_scale;
  const float* bias;
  int gelu;
  const float* residual;
  int64_t ldr;
  int y_bf16;
  void* Y;
  int64_t ldy;
  int kv_col0, kv_width, kv_bf16, page_size;
  void* k_pool;
  void* v_pool;
  const int* wpage;
  const int* woff;
  int ksplit;     // gridDim.z
  int k_per;      // K elements per split (multiple of BK)
  float* partial; // [ksplit][M][N] when ksplit > 1
  // Greedy mode (cbis_gemm_argmax): instead of storing Y, each workgroup
  // writes per row of its tile the tile's top-2 partial {max, second max,
  // index of the max (bits), 0} to amax[row * amax_ld + column tile].
  float4* amax;
  int amax_ld;
  // LayerNorm prologue (skinny kernel, cbis_layernorm_gemm): X is not read;
  // the kernel forms X = LayerNorm(ln_x) row by row, as layernorm_kernel
  // would (same statistics, same rounding), with ln_nch <= kLnMaxChunks.
  const float* ln_x;
  int64_t ln_ldx;
  const float* ln_g;
  const float* ln_b;
  float ln_eps;
  int ln_nch;
  // Every 4-column group of the output is whole and aligned in its
  // destination (Y, the K/V pools or the partials) and in the residual: the
  // parked epilogue then takes its vector path on tiles inside N (with_vec).
  int vec_ok;
  // Tile order of an XCD's contiguous run: N tile fastest when X is the
  // larger operand (its rows are then fetched once per XCD), else M fastest
  // (W's columns are).
  int n_fast;
};

// Tile (m, n) of workgroup bid after xcd_contiguous.
template <int BM, int BN>
__device__ inline int2 tile_of(const GemmArgs& g, int bid) {
  if (g.n_fast) {
    const int nt = (g.N + BN - 1) / BN;
    return make_int2(bid / nt, bid % nt);
  }
  const int mt = (g.M + BM - 1) / BM;
  return make_int2(bid % mt, bid / mt);
}

// g with vec_ok set from its shapes, strides and pointers.
GemmArgs with_vec(const GemmArgs& g) {
  GemmArgs a = g;
  bool ok = (g.N & 3) == 0;
  if (g.ksplit > 1) {
    ok = ok && ((uintptr_t)g.partial & 15u) == 0;
  } else {
    if (g.residual) ok = ok && (g.ldr & 3) == 0 && ((uintptr_t)g.residual & 15u) == 0;
    if (g.k_pool) {
      const uintptr_t al = g.kv_bf16 ? 7u : 15u;
      ok = ok && (g.kv_col0 & 3) == 0 && (g.kv_width & 3) == 0 && ((uintptr_t)g.k_pool & al) == 0 &&
           ((uintptr_t)g.v_pool & al) == 0;
    }
    if (!g.k_pool || g.kv_col0 > 0) ok = ok && (g.ldy & 3) == 0 && ((uintptr_t)g.Y & (g.y_bf16 ? 7u : 15u)) == 0;
  }
  a.vec_ok = ok ? 1 : 0;
  return a;
}
// cbis_layernorm_gemm forms the normalised rows in the skinny kernel for K up
// to kLnPrologueMaxK: every workgroup re-reads its rows' fp32 x and their
// statistics, which costs less than a LayerNorm launch only for short rows
// (config 1, K = 256: 48.6-49.1k -> 50.3-50.4k decode tok/s; config 5,
// K = 2048: 11.00 -> 11.27 ms per step, so there it runs the two kernels).
constexpr int kLnPrologueMaxK = 512;
constexpr int kLnMaxChunks = kLnPrologueMaxK / 256;  // float4 chunks per lane of a row

// Top-2 of a row: the maximum m1 at the lowest index i1 among equal maxima
// (the strict-> scan of src/bench_batching.cpp:66-73), and the largest value
// m2 at any other index (m2 == m1 when the maximum is tied).  NaN never
// wins, except at column 0: the reference's scan starts from the row's first
// value and no comparison with a NaN there succeeds, so a NaN at column 0 is
// the row's answer -- the callers push it as +inf (nan0_as_inf), which wins
// every comparison and keeps the lowest index among equal maxima.  Start
// from m1 = m2 = -inf, i1 = INT_MAX.  top2_push takes one lane's
// columns in increasing order, so a value equal to the maximum never
// displaces it (the strict > keeps the lowest index); a lane that sees only
// -inf keeps i1 = INT_MAX, which the merges rank after every real index.
__device__ inline void top2_push(float& m1, float& m2, int& i1, float v, int c) {
  const bool up = v > m1;
  m2 = fmaxf(m2, up ? m1 : v);
  i1 = up ? c : i1;
  m1 = up ? v : m1;
}
__device__ inline float nan0_as_inf(float v, int c) { return (c == 0 && v != v) ? INFINITY : v; }
// Merges another partial (b1, b2, bi) of disjoint columns; order-free.
__device__ inline void top2_merge(float& m1, float& m2, int& i1, float b1, float b2, int bi) {
  if (b1 > m1 || (b1 == m1 && bi < i1)) {
    m2 = fmaxf(m1, b2);
    m1 = b1;
    i1 = bi;
  } else {
    m2 = fmaxf(m2, b1);
  }
}
// One DPP exchange of a top-2 partial with the partner lane of CTRL.
template <int CTRL>
__device__ inline void top2_dpp(float& m1, float& m2, int& i1) {
  const float b1 = dpp_f32<CTRL>(m1), b2 = dpp_f32<CTRL>(m2);
  const int bi = __builtin_amdgcn_update_dpp(0, i1, CTRL, 0xF, 0xF, true);
  top2_merge(m1, m2, i1, b1, b2, bi);
}
// Every lane of each 16-lane row ends with the row's top-2: partners lane ^ 1,
// lane ^ 2 (quad_perm), the other quad of its 8 (row_half_mirror), the other
// 8 of its 16 (row_mirror) -- each step merges two disjoint lane sets, which
// top2_merge needs (a partial merged with itself would turn its maximum into
// its own second value).  All VALU: no LDS round trip.
__device__ inline void top2_row16(float& m1, float& m2, int& i1) {
  top2_dpp<0xB1>(m1, m2, i1);
  top2_dpp<0x4E>(m1, m2, i1);
  top2_dpp<0x141>(m1, m2, i1);
  top2_dpp<0x140>(m1, m2, i1);
}
// Merges across the lanes l ^ 1, l ^ 2, ... l ^ (W / 2): every lane of a
// W-lane group ends with the group's top-2.
template <int W>
__device__ inline void top2_lanes(float& m1, float& m2, int& i1) {
#pragma unroll
  for (int off = W / 2; off > 0; off >>= 1) {
    const float b1 = __shfl_xor(m1, off, 64), b2 = __shfl_xor(m2, off, 64);
    const int bi = __shfl_xor(i1, off, 64);
    top2_merge(m1, m2, i1, b1, b2, bi);
  }
}

// Exact-form GELU 0.5 v (1 + erf(v / sqrt 2)) (kernels/elementwise.cu:64),
// with erf from Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7):
//   erf(z) = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2),
//   t = 1 / (1 + p z), z >= 0, odd extension for z < 0.
// A dozen VALU ops against the libm erff's range-split polynomial; the GELU
// error it adds (<= 0.75e-7 |v|) is far below the fp32 rounding of the
// GEMM that feeds it.
__device__ inline float gelu_erf(float v) {
  const float z = fabsf(v) * 0.70710678118654752440f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.0f));
  float poly = fmaf(t, 1.061405429f, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f);
  poly *= t;
  const float erf_abs = 1.0f - poly * fast_exp2(-(z * z) * kLog2e);
  return 0.5f * v * (1.0f + copysignf(erf_abs, v));
}

// Applies the epilogue to one accumulator and stores it (the skinny kernel),
// with its inputs loaded beforehand: the channel scale sc, bias bi, residual r
// and the row's K/V slot (wpage * page_size + woff).
__device__ inline void epilogue_store_pre(const GemmArgs& g, int row, int col, float v, float sc, float bi, float r,
                                          int64_t kv_slot) {
  if (g.w_scale) v *= sc;
  if (g.bias) v += bi;
  if (g.gelu) v = gelu_erf(v);
  if (g.residual) v += r;
  if (g.k_pool && col >= g.kv_col0) {
    const int c = col - g.kv_col0;
    const bool is_v = c >= g.kv_width;
    const int e = is_v ? c - g.kv_width : c;
    const int64_t off = kv_slot * g.kv_width + e;
    void* pool = is_v ? g.v_pool : g.k_pool;
    if (g.kv_bf16) ((uint16_t*)pool)[off] = f32_to_bf16(v);
    else ((float*)pool)[off] = v;
    return;
  }
  const int64_t o = (int64_t)row * g.ldy + col;
  if (g.y_bf16) ((uint16_t*)g.Y)[o] = f32_to_bf16(v);
  else ((float*)g.Y)[o] = v;
}

template <typename WT>
struct WLoad;  // global W chunk (covering 16 bytes of LDS) -> uint4 of the compute type
template <>
struct WLoad<float> {
  typedef uint4 raw_t;
  static constexpr int EPC = 4;
  __device__ static inline raw_t load(const float* p) { return *(const uint4*)p; }
  __device__ static inline uint4 cvt(const raw_t& r) { return r; }
};
template <>
struct WLoad<uint16_t> {
  typedef uint4 raw_t;
  static constexpr int EPC = 8;
  __device__ static inline raw_t load(const uint16_t* p) { return *(const uint4*)p; }
  __device__ static inline uint4 cvt(const raw_t& r) { return r; }
};
template <>
struct WLoad<uint8_t> {
  typedef uint2 raw_t;
  static constexpr int EPC = 8;
  __device__ static inline raw_t load(const uint8_t* p) { return *(const uint2*)p; }
  __device__ static inline uint4 cvt(const raw_t& r) {
    uint4 o;
    o.x = (uint32_t)e4m3_to_bf16(r.x & 0xFF) | ((uint32_t)e4m3_to_bf16((r.x >> 8) & 0xFF) << 16);
    o.y = (uint32_t)e4m3_to_bf16((r.x >> 16) & 0xFF) | ((uint32_t)e4m3_to_bf16(r.x >> 24) << 16);
    o.z = (uint32_t)e4m3_to_bf16(r.y & 0xFF) | ((uint32_t)e4m3_to_bf16((r.y >> 8) & 0xFF) << 16);
    o.w = (uint32_t)e4m3_to_bf16((r.y >> 16) & 0xFF) | ((uint32_t)e4m3_to_bf16(r.y >> 24) << 16);
    return o;
  }
};

// Workgroup b is dispatched to XCD b % 8 (measured on gfx950 from the
// XCC_ID hardware register).  Renumbering so that each XCD's workgroups take
// one contiguous run of tiles keeps an XCD on few column blocks of the larger
// operand (tile_of: M fastest for a larger W, N fastest for a larger X), so
// its 4 MB L2 serves the repeats instead of every XCD streaming all of it.
__device__ inline int xcd_contiguous(int bid, int nwg) {
  const int q = nwg >> 3, r = nwg & 7, x = bid & 7;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + (bid >> 3);
}

// LDS image of a 128-byte tile row: 16-byte chunk c of row r sits in slot
// c ^ ((r >> 1) & 7).  gfx950 serves a ds_read_b128 16 lanes (256 bytes, all
// 64 banks) per cycle; the 16 lanes of a fragment load read one chunk of 16
// consecutive rows, i.e. 8 even rows in bytes 0-127 and 8 odd rows in bytes
// 128-255 of the 64 banks, each set in 8 distinct slots: no bank conflicts.
__device__ inline int swz_slot(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }
__device__ inline int swz(int row, int chunk) { return row * 128 + (swz_slot(row, chunk) << 4); }

template <int BM, int BN, int WM, int WN, int FM, int FN>
__device__ inline void epilogue_parked(const GemmArgs& g, int kz, uint8_t* smem, const f32x16_t (&acc)[FM][FN],
                                       int m0, int n0);
// LDS bytes epilogue_parked needs for a BM x BN tile.
template <int BM, int BN>
constexpr int parked_bytes() { return BM * (BN + 8) * 4; }

template <int BM, int BN, int WM, int WN, typename XT, typename WT>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(const GemmArgs g) {
  constexpr bool F32 = sizeof(XT) == 4;
  constexpr int NT = WM * WN * 64;
  constexpr int BK = F32 ? 32 : 64;       // K elements per 128-byte LDS row
  constexpr int XE = F32 ? 4 : 8;         // X elements per 16-byte chunk
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int A_PER = BM * 8 / NT, B_PER = BN * 8 / NT;
  static_assert(A_PER * NT == BM * 8 && B_PER * NT == BN * 8, "tile / thread mismatch");
  typedef WLoad<WT> WL;

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // buffer b: A tile at smem + b*(BM+BN)*128, B tile right after it
  auto lA = [&](int b) { return smem + b * (BM + BN) * 128; };
  auto lB = [&](int b) { return smem + b * (BM + BN) * 128 + BM * 128; };

  // Tile index with XCD-contiguous renumbering.
  const int2 tt = tile_of<BM, BN>(g, xcd_contiguous(blockIdx.x, gridDim.x));
  const int m0 = tt.x * BM, n0 = tt.y * BN;
  const int kz = blockIdx.z;
  const int kbeg = kz * g.k_per;
  const int KT = min(g.k_per, g.K - kbeg) / BK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int half = lane >> 5, l32 = lane & 31;

  const XT* X = (const XT*)g.X;
  const WT* W = (const WT*)g.W;

  uint4 ra[A_PER];
  typename WL::raw_t rb[B_PER];

  auto gload = [&](int kt) {
    const int k0 = kbeg + kt * BK;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int c = tid + i * NT;
      const int r = c >> 3, kc = c & 7;
      const int gr = min(m0 + r, g.M - 1);
      ra[i] = *(const uint4*)(X + (int64_t)gr * g.ldx + k0 + kc * XE);
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = tid + i * NT;
      const int r = c >> 3, kc = c & 7;
      const int gr = min(n0 + r, g.N - 1);
      rb[i] = WL::load(W + (int64_t)gr * g.ldw + k0 + kc * WL::EPC);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int c = tid + i * NT;
      *(uint4*)(lA(buf) + swz(c >> 3, c & 7)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = tid + i * NT;
      *(uint4*)(lB(buf) + swz(c >> 3, c & 7)) = WL::cvt(rb[i]);
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  gload(0);
  lstore(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    const uint8_t* A = lA(buf);
    const uint8_t* B = lB(buf);
    if constexpr (F32) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kc = 2 * j + half;
        f32x4_t af[FM], bf[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i) af[i] = *(const f32x4_t*)(A + swz(wm * TM + i * 32 + l32, kc));
#pragma unroll
        for (int i = 0; i < FN; ++i) bf[i] = *(const f32x4_t*)(B + swz(wn * TN + i * 32 + l32, kc));
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int jj = 0; jj < FN; ++jj)
              acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][e], bf[jj][e], acc[i][jj], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int kc = 2 * ks + half;
        bf16x8_t af[FM], bf[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i) af[i] = *(const bf16x8_t*)(A + swz(wm * TM + i * 32 + l32, kc));
#pragma unroll
        for (int i = 0; i < FN; ++i) bf[i] = *(const bf16x8_t*)(B + swz(wn * TN + i * 32 + l32, kc));
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int jj = 0; jj < FN; ++jj)
            acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[jj], acc[i][jj], 0, 0, 0);
      }
    }
    if (kt + 1 < KT) lstore(buf ^ 1);
    __syncthreads();
  }

  epilogue_parked<BM, BN, WM, WN>(g, kz, smem, acc, m0, n0);
}

// Epilogue of the 4 consecutive output columns col..col+3 (fewer at the
// right edge) handled by one thread: the per-column constants once, then per
// row the inputs (residual, K/V slot) and the finished store.  One 16-byte
// (fp32) or 8-byte (bf16) store when the 4 columns share a destination and
// its alignment allows, else element by element.  The
// wide stores to Y carry the nontemporal hint: every output line is written
// once, by one workgroup, and is read (if at all) by a later kernel (on
// config 2's bf16 M = 4096 shapes 16-byte stores alone gained 11-21%, with
// the hint 30-37%; config 4's fc1 50.0 against 51.7 us).  A call that
// scatters K/V (the QKV projection) stores plainly, Q and K/V alike: the
// step's prefill attention reads them after the decode kernel's non-temporal
// stream over the pools, and plainly stored they are still in the caches then
// (config 4's prefill 17.9 us against 18.2 with Q hinted and 20.3 with Q and
// K/V hinted, same box); so are the split-K partials, which the reduce reads
// right away.
struct Cols4 {
  int col, nc;
  float sc[4], bi[4];
  bool to_kv, vec, res_vec;
  int ce;
  void* pool;

  // raw: the destination is the split-K partials (no epilogue).
  __device__ Cols4(const GemmArgs& g, int col_, bool raw) : col(col_), nc(min(4, g.N - col_)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sc[e] = (!raw && g.w_scale && e < nc) ? g.w_scale[col + e] : 1.f;
      bi[e] = (!raw && g.bias && e < nc) ? g.bias[col + e] : 0.f;
    }
    to_kv = !raw && g.k_pool && col >= g.kv_col0;
    const int c = col - g.kv_col0;
    const bool is_v = to_kv && c >= g.kv_width;
    ce = is_v ? c - g.kv_width : c;
    pool = is_v ? g.v_pool : g.k_pool;
    vec = nc == 4;
    if (raw) {
      vec = vec && (g.N & 3) == 0 && ((uintptr_t)g.partial & 15u) == 0;
    } else if (to_kv) {
      vec = vec && (ce & 3) == 0 && ce + 3 < g.kv_width && ((uintptr_t)pool & (g.kv_bf16 ? 7u : 15u)) == 0 &&
            (g.kv_width & 3) == 0;
    } else {
      vec = vec && (!g.k_pool || col + 3 < g.kv_col0) && (g.ldy & 3) == 0 &&
            ((uintptr_t)g.Y & (g.y_bf16 ? 7u : 15u)) == 0;
    }
    res_vec = g.residual && nc == 4 && (g.ldr & 3) == 0 && ((uintptr_t)g.residual & 15u) == 0;
  }

  // Inputs of one row: residual values and the K/V slot.
  __device__ void load(const GemmArgs& g, int row, float* r, int64_t& slot) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = 0.f;
    slot = 0;
    if (g.residual) {
      const float* rp = g.residual + (int64_t)row * g.ldr + col;
      if (res_vec) {
        const float4 rv = *(const float4*)rp;
        r[0] = rv.x; r[1] = rv.y; r[2] = rv.z; r[3] = rv.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e < nc) r[e] = rp[e];
      }
    }
    if (to_kv) slot = (int64_t)g.wpage[row] * g.page_size + g.woff[row];
  }

  // Scale, bias, GELU, residual, then the store.
  __device__ void finish(const GemmArgs& g, int row, float* v, const float* r, int64_t slot) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = v[e];
      if (g.w_scale) x *= sc[e];
      if (g.bias) x += bi[e];
      if (g.gelu) x = gelu_erf(x);
      if (g.residual) x += r[e];
      v[e] = x;
    }
    if (!vec) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (e >= nc) continue;
        const int cc = col + e;
        if (g.k_pool && cc >= g.kv_col0) {
          const int c2 = cc - g.kv_col0;
          const bool v2 = c2 >= g.kv_width;
          const int64_t off =
              ((int64_t)g.wpage[row] * g.page_size + g.woff[row]) * g.kv_width + (v2 ? c2 - g.kv_width : c2);
          void* pl = v2 ? g.v_pool : g.k_pool;
          if (g.kv_bf16) ((uint16_t*)pl)[off] = f32_to_bf16(v[e]);
          else ((float*)pl)[off] = v[e];
        } else {
          const int64_t o = (int64_t)row * g.ldy + cc;
          if (g.y_bf16) ((uint16_t*)g.Y)[o] = f32_to_bf16(v[e]);
          else ((float*)g.Y)[o] = v[e];
        }
      }
      return;
    }
    const bool bf = to_kv ? g.kv_bf16 : g.y_bf16;
    void* dst = to_kv ? (void*)((char*)pool + (slot * g.kv_width + ce) * (bf ? 2 : 4))
                      : (void*)((char*)g.Y + ((int64_t)row * g.ldy + col) * (bf ? 2 : 4));
    if (g.k_pool) {
      if (bf) *(uint2*)dst = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      else *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
    } else if (bf) {
      const u32x2_t w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      __builtin_nontemporal_store(w, (u32x2_t*)dst);
    } else {
      const f32x4_t w = {v[0], v[1], v[2], v[3]};
      __builtin_nontemporal_store(w, (f32x4_t*)dst);
    }
  }

  // Raw sums to split kz's partials.
  __device__ void store_partial(const GemmArgs& g, int kz, int row, const float* v) const {
    float* pp = g.partial + ((int64_t)kz * g.M + row) * g.N + col;
    if (vec) {
      *(float4*)pp = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < nc) pp[e] = v[e];
    }
  }
};

// Sums the split-K partials (fixed order z = 0, 1, ...) and applies the
// epilogue: one thread per 4 consecutive columns of a row.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const GemmArgs g) {
  const int cgn = (g.N + 3) / 4;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)g.M * cgn) return;
  const int row = (int)(t / cgn), col = (int)(t % cgn) * 4;
  const Cols4 c(g, col, false);
  float r[4];
  int64_t slot;
  c.load(g, row, r, slot);
  const int64_t MN = (int64_t)g.M * g.N;
  const float* pp = g.partial + (int64_t)row * g.N + col;
  const bool pvec = c.nc == 4 && (g.N & 3) == 0 && ((uintptr_t)g.partial & 15u) == 0;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  for (int z = 0; z < g.ksplit; ++z) {
    float p[4] = {0.f, 0.f, 0.f, 0.f};
    if (pvec) {
      const float4 q = *(const float4*)(pp + z * MN);
      p[0] = q.x; p[1] = q.y; p[2] = q.z; p[3] = q.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < c.nc) p[e] = pp[z * MN + e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = z == 0 ? p[e] : v[e] + p[e];
  }
  c.finish(g, row, v, r, slot);
}

inline unsigned splitk_reduce_blocks(const GemmArgs& g) {
  return (unsigned)cdiv((int64_t)g.M * cdiv(g.N, 4), 256);
}

// The split-K reduce fused with the LayerNorm of the finished rows (the
// step's x += fc2(h); xn = LayerNorm(x)): one 256-thread workgroup per row of
// N (a multiple of 4) columns.  The row's float4 chunk i (columns
// 4 (64 i + lane) .. + 3, as in ln_block_row) belongs to wave i % 4, so
// every wave has VPW chunks and all of a thread's loads -- the KS partials,
// bias, residual, gamma, beta -- are issued before its first store.
//
// The results are bit-identical to splitk_reduce_kernel followed by
// layernorm_kernel: each chunk is finished in the reduce's order (partials
// summed z = 0, 1, ..., then bias, then residual) and the row is normalised by
// the same ln_block_row, with layernorm_kernel's chunk count nch.
template <int VPW, int KS, typename LT>
__global__ __launch_bounds__(256) void splitk_layernorm_kernel(const GemmArgs g, const float* __restrict__ lw,
                                                                const float* __restrict__ lb, float eps, int nch,
                                                                LT* __restrict__ ln, int64_t ld_ln) {
  constexpr int NCH = 4 * VPW;
  __shared__ float terms[NCH][64];
  const int row = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int N = g.N;
  const int64_t MN = (int64_t)g.M * N;
  const float* pp = g.partial + (int64_t)row * N;
  const float* rp = g.residual ? g.residual + (int64_t)row * g.ldr : nullptr;
  float4 v[VPW], p[KS - 1][VPW], sc[VPW], bi[VPW], r[VPW], gg[VPW], bb[VPW];
  // (Assignments under if, not conditional expressions: a ?: between a load
  // and a local zero is compiled to a load through a selected pointer, the
  // zero's in scratch memory.)
#pragma unroll
  for (int j = 0; j < VPW; ++j) {
    const int c = ((j * 4 + wave) * 64 + lane) * 4;
    v[j] = bi[j] = r[j] = gg[j] = bb[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    sc[j] = make_float4(1.f, 1.f, 1.f, 1.f);
#pragma unroll
    for (int z = 1; z < KS; ++z) p[z - 1][j] = v[j];
    if (c < N) {
      v[j] = *(const float4*)(pp + c);
#pragma unroll
      for (int z = 1; z < KS; ++z) p[z - 1][j] = *(const float4*)(pp + z * MN + c);
      if (g.w_scale) sc[j] = *(const float4*)(g.w_scale + c);
      if (g.bias) bi[j] = *(const float4*)(g.bias + c);
      if (rp) r[j] = *(const float4*)(rp + c);
      gg[j] = *(const float4*)(lw + c);
      bb[j] = *(const float4*)(lb + c);
    }
  }
#pragma unroll
  for (int j = 0; j < VPW; ++j) {
    const int i = j * 4 + wave;
    const int c = (i * 64 + lane) * 4;
#pragma unroll
    for (int z = 1; z < KS; ++z) {
      v[j].x += p[z - 1][j].x; v[j].y += p[z - 1][j].y; v[j].z += p[z - 1][j].z; v[j].w += p[z - 1][j].w;
    }
    if (g.w_scale) { v[j].x *= sc[j].x; v[j].y *= sc[j].y; v[j].z *= sc[j].z; v[j].w *= sc[j].w; }
    if (g.bias) { v[j].x += bi[j].x; v[j].y += bi[j].y; v[j].z += bi[j].z; v[j].w += bi[j].w; }
    if (rp) { v[j].x += r[j].x; v[j].y += r[j].y; v[j].z += r[j].z; v[j].w += r[j].w; }
    if (c < N) *(float4*)((float*)g.Y + (int64_t)row * g.ldy + c) = v[j];
  }
  ln_block_row<VPW>(v, gg, bb, wave, lane, N, nch, eps, terms, ln + (int64_t)row * ld_ln);
}

// ---------------------------------------------------------------------------
// bf16 x bf16 on a multi-stage LDS ring fed by direct-to-LDS loads.
//
// Each global_load_lds_dwordx4 moves 16 bytes per lane straight from global
// memory into LDS at M0 + 16 * lane (no VGPRs, no ds_write): one wave
// instruction fills 1 KiB = eight 128-byte tile rows.  The chunk swizzle
// (swz_slot) is applied on the global side -- lane i of an instruction
// covering rows 8g..8g+7 fetches the chunk that belongs in slot i & 7 of row
// 8g + (i >> 3) -- so the LDS image is the swizzled layout the ds_read_b128
// fragment loads expect.
//
// STAGES K tiles are in flight: iteration kt waits (s_waitcnt vmcnt) for its
// own tile only, then one barrier, then issues the loads of tile
// kt + STAGES - 1 into the slot that iteration kt - 1 finished reading.
// The loads are issued with inline assembly and waited for explicitly: the
// compiler's own tracking of LDS DMA either waits for every load in flight
// (with a fenced barrier) or misses the wait (with a bare one).  No other
// vector-memory instruction is issued inside the main loop, so the vmcnt
// immediates count exactly the DMA loads of the younger tiles.
// ---------------------------------------------------------------------------
__device__ inline void lds_dma16(const void* gptr, uint32_t lds_addr) {
  // M0 is reserved by the compiler (it never keeps a value there across
  // ordinary code), so it is set right before the load that reads it.
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_addr) : "memory");
}

template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int BM, int BN, int WM, int WN, int STAGES>
__global__ __launch_bounds__(WM* WN * 64) void gemm_bf16_dma_kernel(const GemmArgs g) {
  constexpr int NWAVES = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int ROWS = BM + BN;                 // tile rows per stage (A then B)
  constexpr int GROUPS = ROWS / 8;              // 1 KiB DMA instructions per stage
  constexpr int LPW = GROUPS / NWAVES;          // per wave
  constexpr int STAGE_BYTES = ROWS * 128;
  static_assert(LPW * NWAVES == GROUPS && BM % 8 == 0 && BN % 8 == 0, "tile / wave mismatch");
  static_assert(LPW * (STAGES - 1) < 64, "vmcnt range");

  constexpr int RING = STAGES * STAGE_BYTES;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[RING > parked_bytes<BM, BN>() ? RING : parked_bytes<BM, BN>()];

  const int2 tt = tile_of<BM, BN>(g, xcd_contiguous(blockIdx.x, gridDim.x));
  const int m0 = tt.x * BM, n0 = tt.y * BN;
  const int kz = blockIdx.z;
  const int kbeg = kz * g.k_per;
  const int KT = min(g.k_per, g.K - kbeg) / 64;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int half = lane >> 5, l32 = lane & 31;

  // Per-lane source pointers of this wave's DMA instructions (k tile 0).
  const uint16_t* src[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int grp = wave * LPW + j;
    const int rr = grp * 8 + (lane >> 3);
    const int chunk = swz_slot(rr, lane & 7);  // the chunk that belongs in slot lane & 7 of row rr
    if (rr < BM) {
      const int r = min(m0 + rr, g.M - 1);
      src[j] = (const uint16_t*)g.X + (int64_t)r * g.ldx + kbeg + chunk * 8;
    } else {
      const int r = min(n0 + rr - BM, g.N - 1);
      src[j] = (const uint16_t*)g.W + (int64_t)r * g.ldw + kbeg + chunk * 8;
    }
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  const uint32_t wave_lds = __builtin_amdgcn_readfirstlane(lds0 + wave * LPW * 1024);

  auto issue = [&](int kt) {
    const uint32_t base = wave_lds + (uint32_t)((kt % STAGES) * STAGE_BYTES);
#pragma unroll
    for (int j = 0; j < LPW; ++j) lds_dma16(src[j] + kt * 64, base + j * 1024);
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment byte offsets inside a stage: swz(row, kc); every fragment row
  // this lane reads is l32 plus a multiple of 32, so its swizzle key is l32's.
  const int a_row0 = (wm * TM + l32) * 128;
  const int b_row0 = (BM + wn * TN + l32) * 128;
  const int sw = (l32 >> 1) & 7;
  bf16x8_t af[2][FM], bf[2][FN];
  auto load_frags = [&](int slot, int ks, int fb) {
    const uint8_t* st = smem + slot * STAGE_BYTES;
    const int kc = ((2 * ks + half) ^ sw) << 4;
#pragma unroll
    for (int i = 0; i < FM; ++i) af[fb][i] = *(const bf16x8_t*)(st + a_row0 + i * 32 * 128 + kc);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[fb][j] = *(const bf16x8_t*)(st + b_row0 + j * 32 * 128 + kc);
  };
  // Waits until k tile t has landed in LDS for every wave: at most
  // (last - t) * LPW of this wave's DMA loads may remain (tiles t+1..last are
  // the younger ones in flight), then a barrier.  The lgkmcnt wait makes
  // every wave's earlier ds_reads complete before any wave refills the slot
  // they read.
  auto await_tile = [&](int t, int last) {
    const int younger = last - t;
    if constexpr (STAGES >= 4) {
      if (younger >= 3) wait_vmcnt<3 * LPW>();
      else if (younger == 2) wait_vmcnt<2 * LPW>();
      else if (younger == 1) wait_vmcnt<LPW>();
      else wait_vmcnt<0>();
    } else {
      if (younger >= 2) wait_vmcnt<2 * LPW>();
      else if (younger == 1) wait_vmcnt<LPW>();
      else wait_vmcnt<0>();
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
  };

  // Tiles 0..STAGES-1 in flight, one per slot.
#pragma unroll
  for (int t = 0; t < STAGES; ++t)
    if (t < KT) issue(t);
  await_tile(0, min(KT - 1, STAGES - 1));
  load_frags(0, 0, 0);

  // The fragments of sub-step ks+1 are read while sub-step ks's MFMAs run;
  // across a tile boundary the barrier sits between the last sub-step's
  // fragment reads and its MFMAs, and the freed slot is refilled with tile
  // kt + STAGES right after it.
  for (int kt = 0; kt < KT; ++kt) {
    const int slot = kt % STAGES;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int fb = ks & 1;
      if (ks < 3) {
        load_frags(slot, ks + 1, fb ^ 1);
      } else if (kt + 1 < KT) {
        await_tile(kt + 1, min(KT - 1, kt + STAGES - 1));
        if (kt + STAGES < KT) issue(kt + STAGES);
        load_frags((kt + 1) % STAGES, 0, fb ^ 1);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[fb][i], bf[fb][j], acc[i][j], 0, 0, 0);
    }
  }

  epilogue_parked<BM, BN, WM, WN>(g, kz, smem, acc, m0, n0);
}

template <int BM, int BN, int WM, int WN, int STAGES>
int launch_dma(const GemmArgs& g, hipStream_t s) {
  const int64_t tiles = cdiv(g.M, BM) * cdiv(g.N, BN);
  gemm_bf16_dma_kernel<BM, BN, WM, WN, STAGES><<<dim3((unsigned)tiles, 1, g.ksplit), WM * WN * 64, 0, s>>>(with_vec(g));
  return check_launch("cbis_gemm(bf16)");
}

// ---------------------------------------------------------------------------
// bf16 x bf16, wave-specialised, for grids of at least half a CU count of
// 128 x 128 tiles.
//
// 8 waves, one workgroup per CU.  Waves 0-3 (one per SIMD) are consumers:
// they only read fragments from LDS and issue MFMAs, each on a
// (BM/WM) x (BN/(4/WM)) sub-tile (2 x 2, or 1 x 4 for 160-row tiles).
// Waves 4-7 are producers: they only issue the
// direct-to-LDS loads of a STAGES-slot ring (same row layout and swizzle as
// gemm_bf16_dma_kernel) and wait for them, so a load that stalls at issue
// (the texture path takes a 1 KiB DMA instruction per ~16 cycles per CU)
// never holds back an MFMA.  One barrier per K tile: before barrier t the
// producers have waited (vmcnt) for tile t and the consumers have finished
// their ds_reads of tile t - 1, whose slot the producers refill with tile
// t - 1 + STAGES right after it.  With REGS > 0 the producers instead load
// into a REGS-deep ring of VGPRs (they have the registers the consumers need,
// unused) and ds_write each tile into its slot, so a 2-slot ring (64 KiB at
// 128 x 128) is enough and two workgroups share a CU.
//
// After the K loop the consumers park their accumulators in LDS as a
// row-major fp32 tile (the ring is free by then; a tile too large for LDS is
// parked in two row blocks, one after the other) and all 8 waves apply the
// epilogue row by row, 4 consecutive columns per thread: the channel scale
// and bias are loaded once per thread, residual / partial accesses are 16
// bytes and bf16 / K/V stores 8 bytes; on aligned tiles inside N every
// global input of the thread's rows is loaded before its first store
// (epilogue_rows_vec), elsewhere the inputs of 2-4 rows before their stores
// (Y may alias the residual either way).
// ---------------------------------------------------------------------------
constexpr int kWsProducers = 4;

template <int BM, int BN, int STAGES, int WM>
struct WsTile {
  static constexpr int WN = 4 / WM;                    // consumers as WM x WN
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 32, FN = TN / 32;
  static constexpr int ROWS = BM + BN;
  static constexpr int LPW = ROWS / 8 / kWsProducers;  // 1 KiB DMA instructions per producer per tile
  static constexpr int STAGE_BYTES = ROWS * 128;
  static constexpr int RING = STAGES * STAGE_BYTES;
  static constexpr int PITCH = BN + 8;                 // floats per parked output row
  static constexpr int kLdsMax = 160 * 1024;
  // The accumulators are parked PH row blocks at a time when the whole tile
  // does not fit.
  static constexpr int PH = BM * PITCH * 4 <= kLdsMax ? 1 : (BM / 2) * PITCH * 4 <= kLdsMax ? 2 : 4;
  static constexpr int PR = BM / PH;                   // rows per parked block
  static constexpr int PARK = PR * PITCH * 4;
  static constexpr int LDS = RING > PARK ? RING : PARK;
  static_assert(WM * WN == 4 && TM % 32 == 0 && TN % 32 == 0, "consumer layout");
  static_assert(LPW * 8 * kWsProducers == ROWS, "tile rows / producers");
  static_assert(LPW * (STAGES - 1) < 64, "vmcnt range");
  static_assert(BM % PH == 0 && PR * PITCH * 4 <= kLdsMax && LDS <= kLdsMax, "LDS");
};

// Vector path of epilogue_rows, for tiles whose every 4-column group is whole
// and aligned in its destination (g.vec_ok, tile inside N).  vmcnt counts
// stores as well as loads and retires them in order, so a memory read issued
// after a store -- or a register that an in-flight store still names being
// rewritten on a load's path -- makes the code wait for that store's write
// acknowledgement; the general path's per-row loads and branches cost such a
// wait on every row.  Here the thread's global inputs (RES: the residual
// values, KV: the rows' page and offset ids) are all loaded before the first
// store, the parked values are read G rows at a time from LDS (which vmcnt
// does not count), and each row is finished -- the same operations in the
// same order as Cols4::finish -- and stored with one 16-byte (fp32) or 8-byte
// (bf16) store.  RES and KV are template flags so that a variant holds only
// the registers its inputs need.  Config 4's step, same box: qkv 41.3 ->
// 37.2 us, out-projection 25.7 -> 22.9, fc1 50.2 -> 48.5 (its GELU is most of
// what remains of its epilogue).
template <int PASSES, int RPP, bool RES, bool KV>
__device__ inline void epilogue_rows_vec(const GemmArgs& g, int kz, const float* tile, int pitch, int m0, int n0,
                                         int cg, int rs) {
  constexpr int G = PASSES % 4 == 0 ? 4 : (PASSES % 2 == 0 ? 2 : 1);
  const bool raw = g.ksplit > 1;  // RES and KV imply !raw
  const int col = n0 + 4 * cg;
  float sc[4], bi[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    sc[e] = (!raw && g.w_scale) ? g.w_scale[col + e] : 1.f;
    bi[e] = (!raw && g.bias) ? g.bias[col + e] : 0.f;
  }
  const bool to_kv = KV && col >= g.kv_col0;
  const int c = col - g.kv_col0;
  const bool is_v = to_kv && c >= g.kv_width;
  const bool bf = !raw && (to_kv ? g.kv_bf16 : g.y_bf16);
  const int esz = bf ? 2 : 4;
  // Destination of row index ri (the row, or the K/V slot): base + ri * stride.
  char* base;
  int64_t stride;
  if (raw) {
    base = (char*)(g.partial + (int64_t)kz * g.M * g.N + col);
    stride = (int64_t)g.N * 4;
  } else if (to_kv) {
    base = (char*)(is_v ? g.v_pool : g.k_pool) + (int64_t)(is_v ? c - g.kv_width : c) * esz;
    stride = (int64_t)g.kv_width * esz;
  } else {
    base = (char*)g.Y + (int64_t)col * esz;
    stride = g.ldy * esz;
  }
  // Rows clamped to M - 1 (rows past M are not stored), so the loads need no
  // per-lane condition and issue back to back.
  float4 res[RES ? PASSES : 1];
  uint32_t wp[KV ? PASSES : 1], wo[KV ? PASSES : 1];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int row = min(m0 + p * RPP + rs, g.M - 1);
    if constexpr (RES) res[p] = *(const float4*)(g.residual + (int64_t)row * g.ldr + col);
    if constexpr (KV) {
      wp[p] = (uint32_t)g.wpage[row];
      wo[p] = (uint32_t)g.woff[row];
    }
  }
  const bool hs = !raw && g.w_scale, hb = !raw && g.bias, hg = !raw && g.gelu;
#pragma unroll
  for (int p0 = 0; p0 < PASSES; p0 += G) {
    float4 tv[G];
#pragma unroll
    for (int q = 0; q < G; ++q) tv[q] = *(const float4*)(tile + ((p0 + q) * RPP + rs) * pitch + 4 * cg);
#pragma unroll
    for (int q = 0; q < G; ++q) {
      const int p = p0 + q;
      const int row = m0 + p * RPP + rs;
      float v[4] = {tv[q].x, tv[q].y, tv[q].z, tv[q].w};
      // Scale and bias by selects (x * 1 or x + 0 would not be exact for
      // every x), GELU under one branch per row.
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float xs = v[e] * sc[e];
        v[e] = hs ? xs : v[e];
        const float xb = v[e] + bi[e];
        v[e] = hb ? xb : v[e];
      }
      if (hg) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gelu_erf(v[e]);
      }
      if constexpr (RES) {
        v[0] += res[p].x; v[1] += res[p].y; v[2] += res[p].z; v[3] += res[p].w;
      }
      // Slot ids are non-negative: widened unsigned, so no sign extension is
      // computed (and waited for) right after their loads.
      int64_t ri = row;
      if constexpr (KV) {
        if (to_kv) ri = (int64_t)((uint64_t)wp[p] * (uint32_t)g.page_size + wo[p]);
      }
      char* dst = base + ri * stride;
      if (row >= g.M) continue;
      if (raw || KV) {
        // Split-K partials and calls that scatter K/V: plain stores.
        if (bf) *(uint2*)dst = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        else *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
      } else if (bf) {
        const u32x2_t w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        __builtin_nontemporal_store(w, (u32x2_t*)dst);
      } else {
        const f32x4_t w = {v[0], v[1], v[2], v[3]};
        __builtin_nontemporal_store(w, (f32x4_t*)dst);
      }
    }
  }
}

// Epilogue over a parked BM x BN fp32 tile by the workgroup's NT threads:
// thread (rs, cg) takes columns 4cg..4cg+3 of rows rs, rs + RPP, ...; the
// inputs of 4 rows are loaded before their stores (Y may alias the residual).
template <int BM, int BN, int NT = 512>
__device__ inline void epilogue_rows(const GemmArgs& g, int kz, const float* tile, int pitch, int m0, int n0,
                                     int tid) {
  constexpr int CG = BN / 4;      // 4-column groups per row
  constexpr int RPP = NT / CG;    // rows per pass
  constexpr int PASSES = BM / RPP;
  constexpr int G = PASSES % 4 == 0 ? 4 : 2;  // rows whose inputs are loaded before their stores
  static_assert(RPP * CG == NT && PASSES % G == 0, "epilogue thread map");
  const int cg = tid % CG, rs = tid / CG;
  // The vector path (tiles inside N with aligned groups); a residual is
  // preloaded there only for up to 8 rows per thread (its registers would
  // otherwise raise every call's allocation), and never with a K/V scatter.
  if (g.vec_ok && n0 + BN <= g.N) {
    const bool raw_call = g.ksplit > 1, res = !raw_call && g.residual, kv = !raw_call && g.k_pool;
    if (!res && !kv) {
      epilogue_rows_vec<PASSES, RPP, false, false>(g, kz, tile, pitch, m0, n0, cg, rs);
      return;
    }
    if (!res) {
      epilogue_rows_vec<PASSES, RPP, false, true>(g, kz, tile, pitch, m0, n0, cg, rs);
      return;
    }
    if constexpr (PASSES <= 8) {
      if (!kv) {
        epilogue_rows_vec<PASSES, RPP, true, false>(g, kz, tile, pitch, m0, n0, cg, rs);
        return;
      }
    }
  }
  if (n0 + 4 * cg >= g.N) return;
  const bool raw = g.ksplit > 1;
  const Cols4 c(g, n0 + 4 * cg, raw);
#pragma unroll 1
  for (int p0 = 0; p0 < PASSES; p0 += G) {
    float v[G][4], r[G][4];
    int64_t slot[G];
#pragma unroll
    for (int q = 0; q < G; ++q) {
      const int lr = (p0 + q) * RPP + rs;
      const float4 t = *(const float4*)(tile + lr * pitch + 4 * cg);
      v[q][0] = t.x; v[q][1] = t.y; v[q][2] = t.z; v[q][3] = t.w;
      if (!raw && m0 + lr < g.M) c.load(g, m0 + lr, r[q], slot[q]);
    }
#pragma unroll
    for (int q = 0; q < G; ++q) {
      const int row = m0 + (p0 + q) * RPP + rs;
      if (row >= g.M) continue;
      if (raw) c.store_partial(g, kz, row, v[q]);
      else c.finish(g, row, v[q], r[q], slot[q]);
    }
  }
}

// Epilogue of the single-role kernels (gemm_kernel, gemm_bf16_dma_kernel):
// every wave parks its accumulators in LDS as one row-major fp32 tile
// (pitch BN + 8: the two row halves of a 32 x 32 block, 4 rows apart, land
// in opposite halves of the 64 banks) and the whole workgroup runs
// epilogue_rows over it.  Stored straight from the MFMA layout, a wave's
// store instruction covers 2 rows x 128 bytes (4 bytes a lane); from the
// parked tile it covers 4-8 rows x 256-512 bytes (16 bytes a lane), a
// quarter of the instructions for the same bytes.  smem needs
// BM * (BN + 8) * 4 bytes; the caller's K loop must be done with it.
template <int BM, int BN, int WM, int WN, int FM, int FN>
__device__ inline void epilogue_parked(const GemmArgs& g, int kz, uint8_t* smem, const f32x16_t (&acc)[FM][FN],
                                       int m0, int n0) {
  constexpr int TM = BM / WM, TN = BN / WN, PITCH = BN + 8;
  static_assert(FM * 32 == TM && FN * 32 == TN, "accumulator blocks");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int half = lane >> 5, l32 = lane & 31;
  float* tile = (float*)smem;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        tile[(wm * TM + i * 32 + 8 * (e >> 2) + 4 * half + (e & 3)) * PITCH + wn * TN + j * 32 + l32] = acc[i][j][e];
  __syncthreads();
  epilogue_rows<BM, BN, WM * WN * 64>(g, kz, tile, PITCH, m0, n0, tid);
}

// Channel scale and bias of the greedy epilogue's columns for lane j of a
// 16-lane row group: columns n0 + 64 k + 4 j + e (loaded once per tile, with
// the column clamped to N - 1: columns past N are never ranked).
template <int BN>
struct Top2Cols {
  static constexpr int KC = BN / 64;  // float4 chunks per lane
  float sc[KC][4], bi[KC][4];
  __device__ Top2Cols(const GemmArgs& g, int n0, int j) {
#pragma unroll
    for (int k = 0; k < KC; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = min(n0 + 64 * k + 4 * j + e, g.N - 1);
        sc[k][e] = g.w_scale ? g.w_scale[c] : 1.f;
        bi[k][e] = g.bias ? g.bias[c] : 0.f;
      }
  }
};
struct NoCols {
  __device__ NoCols(const GemmArgs&, int, int) {}
};

// Greedy-mode epilogue over a parked BM x BN fp32 tile: each 16-lane row of
// a wave takes one tile row (a wave 4 rows at a time), lane j of it the
// columns 4 j + 64 k .. + 3 (16-byte LDS reads, the 16 lanes covering 256
// consecutive bytes: no bank conflicts); each value gets the channel scale
// and bias exactly as Cols4::finish applies them (so it equals the logit the
// store path would write); the row's top-2 over the tile's columns is
// written for column tile n0 / BN.  The work is VALU-bound, so the variants
// for a tile inside N (CHECK false: no column test) and for calls without
// scale or bias (AFFINE false) are separate loops, chosen once per tile; the
// partials of all the wave's rows are stored after the last of them is
// formed, so no store is waited for inside the epilogue (config 4's lm_head
// in the step, same box: 188 -> 164.5 us, 969 TFLOP/s).
template <int BM, int BN, int NT, bool CHECK, bool AFFINE>
__device__ inline void epilogue_top2_rows(const GemmArgs& g, const Top2Cols<BN>& cc, const float* tile, int pitch,
                                          int m0, int n0, int tid) {
  constexpr int KC = Top2Cols<BN>::KC;
  static_assert(KC * 64 == BN && BM % 4 == 0, "epilogue_top2 tile");
  constexpr int RPI = 4 * (NT / 64);  // rows per iteration of the workgroup
  constexpr int IT = (BM + RPI - 1) / RPI;
  const int wave = tid >> 6, lane = tid & 63, grp = lane >> 4, j = lane & 15;
  const bool hs = g.w_scale != nullptr, hb = g.bias != nullptr;
  float4 part[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int rw = 4 * wave + RPI * it;  // the wave's first row: wave-uniform
    float m1 = -INFINITY, m2 = -INFINITY;
    int i1 = 0x7FFFFFFF;
    if (rw < BM) {
      const int r = rw + grp;
      float4 t[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k) t[k] = *(const float4*)(tile + r * pitch + 64 * k + 4 * j);
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const float tv[4] = {t[k].x, t[k].y, t[k].z, t[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = n0 + 64 * k + 4 * j + e;
          float v = tv[e];
          if constexpr (AFFINE) {
            const float xs = v * cc.sc[k][e];
            v = hs ? xs : v;
            const float xb = v + cc.bi[k][e];
            v = hb ? xb : v;
          }
          if constexpr (CHECK) v = c < g.N ? v : -INFINITY;  // -inf: no effect on the top-2
          if (k == 0 && e == 0) v = nan0_as_inf(v, c);       // only lane 0 of the first tile holds column 0
          top2_push(m1, m2, i1, v, c);
        }
      }
    }
    top2_row16(m1, m2, i1);
    part[it] = make_float4(m1, m2, __int_as_float(i1), 0.f);
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int r = 4 * wave + RPI * it + grp;
    if (j == 0 && 4 * wave + RPI * it < BM && m0 + r < g.M)
      g.amax[(int64_t)(m0 + r) * g.amax_ld + n0 / BN] = part[it];
  }
}

template <int BM, int BN, int NT = 512>
__device__ inline void epilogue_top2(const GemmArgs& g, const Top2Cols<BN>& cc, const float* tile, int pitch, int m0,
                                     int n0, int tid) {
  const bool check = n0 + BN > g.N, affine = g.w_scale || g.bias;
  if (check) epilogue_top2_rows<BM, BN, NT, true, true>(g, cc, tile, pitch, m0, n0, tid);
  else if (affine) epilogue_top2_rows<BM, BN, NT, false, true>(g, cc, tile, pitch, m0, n0, tid);
  else epilogue_top2_rows<BM, BN, NT, false, false>(g, cc, tile, pitch, m0, n0, tid);
}

template <int BM, int BN, int STAGES, int REGS, int WM, bool TOP2>
__global__ __launch_bounds__(512) void gemm_bf16_ws_kernel(const GemmArgs g) {
  typedef WsTile<BM, BN, STAGES, WM> T;
  constexpr int LPW = T::LPW, STAGE_BYTES = T::STAGE_BYTES, FM = T::FM, FN = T::FN;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[T::LDS];

  const int2 tt = tile_of<BM, BN>(g, xcd_contiguous(blockIdx.x, gridDim.x));
  const int m0 = tt.x * BM, n0 = tt.y * BN;
  const int kz = blockIdx.z;
  const int kbeg = kz * g.k_per;
  const int KT = min(g.k_per, g.K - kbeg) / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;  // consumer sub-tile (waves 0-3)
  const int half = lane >> 5, l32 = lane & 31;
  f32x16_t acc[FM][FN];

  if (wave >= 4) {
    // Producer: tile rows p*8*LPW .. of every stage (A rows first, then B).
    const int p = wave - 4;
    const uint16_t* src[LPW];
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int rr = (p * LPW + j) * 8 + (lane >> 3);
      const int chunk = swz_slot(rr, lane & 7);  // the chunk that belongs in slot lane & 7 of row rr
      if (rr < BM) src[j] = (const uint16_t*)g.X + (int64_t)min(m0 + rr, g.M - 1) * g.ldx + kbeg + chunk * 8;
      else src[j] = (const uint16_t*)g.W + (int64_t)min(n0 + rr - BM, g.N - 1) * g.ldw + kbeg + chunk * 8;
    }
    if constexpr (REGS == 0) {
      const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
      const uint32_t wave_lds = __builtin_amdgcn_readfirstlane(lds0 + p * LPW * 1024);
      auto issue = [&](int kt) {
        const uint32_t base = wave_lds + (uint32_t)((kt % STAGES) * STAGE_BYTES);
#pragma unroll
        for (int j = 0; j < LPW; ++j) lds_dma16(src[j] + kt * 64, base + j * 1024);
      };
      // Waits for a tile with `younger` tiles issued after it.
      auto wait_tile = [&](int younger) {
        if constexpr (STAGES >= 4) {
          if (younger >= 3) { wait_vmcnt<3 * LPW>(); return; }
        }
        if constexpr (STAGES >= 3) {
          if (younger >= 2) { wait_vmcnt<2 * LPW>(); return; }
        }
        if (younger >= 1) wait_vmcnt<LPW>();
        else wait_vmcnt<0>();
      };
#pragma unroll
      for (int t = 0; t < STAGES; ++t)
        if (t < KT) issue(t);
      wait_tile(min(KT - 1, STAGES - 1));
      asm volatile("s_barrier" ::: "memory");
      for (int kt = 0; kt + 1 < KT; ++kt) {
        wait_tile(min(KT - 1, kt + STAGES - 1) - (kt + 1));
        asm volatile("s_barrier" ::: "memory");
        if (kt + STAGES < KT) issue(kt + STAGES);
      }
      wait_vmcnt<0>();
    } else {
      // Register-staged: tiles go global -> VGPRs (a REGS-deep ring, the
      // compiler waits for each load where its ds_write uses it) -> LDS.
      // After barrier j the slot of tile j - 1 is free and receives tile
      // j + STAGES - 1, whose registers are refilled with tile
      // j + STAGES - 1 + REGS; its ds_writes finish before barrier j + 1.
      static_assert(STAGES >= 2 && STAGES - 1 <= REGS, "register ring shorter than the LDS lead");
      u32x4_t regs[REGS][LPW];
      uint8_t* my_lds = smem + p * LPW * 1024 + lane * 16;
      auto load = [&](int r, int t) {
#pragma unroll
        for (int j = 0; j < LPW; ++j) regs[r][j] = *(const u32x4_t*)(src[j] + t * 64);
      };
      auto store = [&](int r, int t) {
#pragma unroll
        for (int j = 0; j < LPW; ++j) *(u32x4_t*)(my_lds + (t % STAGES) * STAGE_BYTES + j * 1024) = regs[r][j];
      };
#pragma unroll
      for (int r = 0; r < REGS; ++r)
        if (r < KT) load(r, r);
#pragma unroll
      for (int t = 0; t < STAGES - 1; ++t)
        if (t < KT) {
          store(t % REGS, t);
          if (t + REGS < KT) load(t % REGS, t + REGS);
        }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      for (int j0 = 0; j0 < KT; j0 += REGS) {
#pragma unroll
        for (int r = 0; r < REGS; ++r) {
          const int j = j0 + r;
          if (j >= KT) break;
          const int t = j + STAGES - 1;
          constexpr int kLead = STAGES - 1;
          const int rs = (r + kLead) % REGS;  // t % REGS: j0 is a multiple of REGS
          if (t < KT) {
            store(rs, t);
            if (t + REGS < KT) load(rs, t + REGS);
          }
          if (j + 1 < KT) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
      }
    }
    asm volatile("s_barrier" ::: "memory");  // consumers done with the ring
  } else {
    // Consumer: sub-tile (wm, wn) of WM x (4 / WM).
    __builtin_amdgcn_s_setprio(2);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const int a_row0 = (wm * T::TM + l32) * 128;
    const int b_row0 = (BM + wn * T::TN + l32) * 128;
    const int sw = (l32 >> 1) & 7;  // swizzle key of every fragment row this lane reads
    bf16x8_t af[2][FM], bf[2][FN];
    auto load_frags = [&](int slot, int ks, int fb) {
      const uint8_t* st = smem + slot * STAGE_BYTES;
      const int kc = ((2 * ks + half) ^ sw) << 4;
#pragma unroll
      for (int i = 0; i < FM; ++i) af[fb][i] = *(const bf16x8_t*)(st + a_row0 + i * 32 * 128 + kc);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[fb][j] = *(const bf16x8_t*)(st + b_row0 + j * 32 * 128 + kc);
    };
    asm volatile("s_barrier" ::: "memory");
    load_frags(0, 0, 0);
    for (int kt = 0; kt < KT; ++kt) {
      const int slot = kt % STAGES;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int fb = ks & 1;
        if (ks < 3) {
          load_frags(slot, ks + 1, fb ^ 1);
        } else if (kt + 1 < KT) {
          asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
          load_frags((kt + 1) % STAGES, 0, fb ^ 1);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[fb][i], bf[fb][j], acc[i][j], 0, 0, 0);
        // Issue the next sub-step's fragment reads between this sub-step's
        // MFMAs, one read after each MFMA, so they land while the MFMAs run
        // (left to itself the scheduler sinks them below the MFMAs and the
        // next sub-step waits on them: qkv 41.3 -> 40.1 us, fc1 50.4 -> 48.5).
        constexpr int kReads = FM + FN, kMfma = FM * FN, kPairs = kReads < kMfma ? kReads : kMfma;
#pragma unroll
        for (int q = 0; q < kPairs; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        }
        if constexpr (kMfma > kPairs) __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kPairs, 0);
        if constexpr (kReads > kPairs) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPairs, 0);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // done with the ring
  }
  // Park the accumulators (PH blocks of PR rows) and finish them row-wise.
  float* park = (float*)smem;
  // Greedy mode: the tile's column constants, loaded once for all row blocks.
  const typename std::conditional<TOP2, Top2Cols<BN>, NoCols>::type cols(g, n0, tid & 15);
#pragma unroll
  for (int h = 0; h < T::PH; ++h) {
    if (wave < 4) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int r = wm * T::TM + i * 32 + 8 * (e >> 2) + 4 * half + (e & 3) - h * T::PR;
            if (T::PH == 1 || (r >= 0 && r < T::PR)) park[r * T::PITCH + wn * T::TN + j * 32 + l32] = acc[i][j][e];
          }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // Greedy mode is a separate instantiation: the two epilogues in one kernel
    // raised its scalar-register spills (24 -> 157 at 160 x 256) and slowed
    // the K loop of every call.
    if constexpr (TOP2) epilogue_top2<T::PR, BN>(g, cols, (const float*)smem, T::PITCH, m0 + h * T::PR, n0, tid);
    else epilogue_rows<T::PR, BN>(g, kz, (const float*)smem, T::PITCH, m0 + h * T::PR, n0, tid);
    if (h + 1 < T::PH) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
}

template <int BM, int BN, int STAGES, int REGS = 0, int WM = 2>
int launch_ws(const GemmArgs& g, hipStream_t s) {
  const int64_t tiles = cdiv(g.M, BM) * cdiv(g.N, BN);
  if (g.amax) gemm_bf16_ws_kernel<BM, BN, STAGES, REGS, WM, true><<<dim3((unsigned)tiles, 1, 1), 512, 0, s>>>(g);
  else gemm_bf16_ws_kernel<BM, BN, STAGES, REGS, WM, false><<<dim3((unsigned)tiles, 1, g.ksplit), 512, 0, s>>>(with_vec(g));
  return check_launch("cbis_gemm(bf16 ws)");
}

// ---------------------------------------------------------------------------
// Skinny GEMM for M <= 64 rows (decode steps): weight-streaming on MFMA.
//
// A workgroup of 8 waves owns 16 output columns; the waves split K into 8
// contiguous ranges and each streams its W slice straight into MFMA B
// operands (no LDS staging: every W element is used by all M rows of one
// MFMA), with the X fragments coming from L2.  The 8 partial 16-column
// tiles are summed through LDS and wave 0 applies the epilogue.
//   bf16 X:  v_mfma_f32_16x16x32_bf16, lane l holds 8 consecutive k of row
//            (or W row) l % 16 at k offset 8 * (l / 16); fp8 W is widened
//            to bf16 with v_cvt_scalef32_pk_bf16_fp8 (scale 1: exact, every
//            e4m3 value is a bf16 value), the channel scale is applied in
//            the epilogue;
//   fp32 X:  v_mfma_f32_16x16x4_f32, lane l holds k = 4 * (l / 16) + e of a
//            16-k block in element e of a float4, one MFMA per e.
// C fragment: lane l holds rows 4 * (l / 16) + i, column l % 16.
// ---------------------------------------------------------------------------
template <typename WT>
struct SkinnyW;
template <>
struct SkinnyW<uint16_t> {  // bf16: 8 elements = 16 bytes
  __device__ static inline bf16x8_t load(const uint16_t* p) { return *(const bf16x8_t*)p; }
};
template <>
struct SkinnyW<uint8_t> {  // fp8 e4m3: 8 elements = 8 bytes
  __device__ static inline bf16x8_t load(const uint8_t* p) {
    const uint2 r = *(const uint2*)p;
    return load_pair(r.x, r.y);
  }
  // 8 e4m3 codes (two dwords, lowest byte first) -> 8 bf16.
  __device__ static inline bf16x8_t load_pair(uint32_t lo, uint32_t hi) {
    const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    uint4 u;
    u.x = __builtin_bit_cast(uint32_t, a);
    u.y = __builtin_bit_cast(uint32_t, b);
    u.z = __builtin_bit_cast(uint32_t, c);
    u.w = __builtin_bit_cast(uint32_t, d);
    return __builtin_bit_cast(bf16x8_t, u);
  }
};

constexpr int kSkinnyWaves = 8;

template <typename XT, typename WT, int MB, bool LN>
__global__ __launch_bounds__(kSkinnyWaves * 64) void gemm_skinny_kernel(const GemmArgs g) {
  constexpr bool F32 = sizeof(XT) == 4;
  constexpr int KB = F32 ? 16 : 32;  // k per MFMA step
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = min(n0 + c16, g.N - 1);
  // Split-K (g.partial set, grid.y = g.ksplit): workgroup (x, z) sums K range
  // [z k_per, (z + 1) k_per) and stores the raw sums as partial z; the
  // epilogue then runs in the reduce.  Unsplit, k_per = K.
  const int64_t kofs = (int64_t)blockIdx.y * g.k_per;
  const int nkb = g.k_per / KB;
  const int kb0 = (nkb * wave) / kSkinnyWaves, kb1 = (nkb * (wave + 1)) / kSkinnyWaves;

  f32x4_t acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  int xrow[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) xrow[i] = min(i * 16 + c16, g.M - 1);

  // Wave 0 finishes the tile.  With up to 32 rows (MB <= 2) it loads the
  // epilogue's inputs (channel scale, bias, residual, K/V slots of its rows)
  // now, so their round trip overlaps the K loop instead of following it;
  // rows / columns past M / N read row M - 1 / column N - 1 (in bounds, never
  // stored).  At MB = 4 the registers they would hold through the K loop
  // cost more (spills), so there they are loaded after it.
  constexpr bool PRE = MB <= 2;
  const int pcol = min(n0 + c16, g.N - 1);
  float pre_sc = 1.f, pre_bi = 0.f;
  float pre_r[MB][4];
  int64_t pre_slot[MB][4];
  auto load_pre = [&]() {
    if (g.w_scale) pre_sc = g.w_scale[pcol];
    if (g.bias) pre_bi = g.bias[pcol];
    const bool kv = g.k_pool && pcol >= g.kv_col0;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = min(i * 16 + 4 * q + e, g.M - 1);
        pre_r[i][e] = g.residual ? g.residual[(int64_t)row * g.ldr + pcol] : 0.f;
        pre_slot[i][e] = kv ? (int64_t)g.wpage[row] * g.page_size + g.woff[row] : 0;
      }
  };
  if (PRE && wave == 0 && !g.amax && !g.partial) load_pre();

  // LayerNorm prologue: each wave takes rows wave, wave + 8, ... of the
  // workgroup's 16 MB rows and forms their mean and 1/std exactly as
  // ln_block_row does (per-lane sums over the row's float4 chunks 0 .. nch-1
  // in order, then wave_sum; no FMA contraction in either), so the
  // normalised X equals layernorm_kernel's output bit for bit.  Rows past M
  // repeat row M - 1.
  __shared__ float ln_mu[16 * MB], ln_rs[16 * MB];
  float lnm[MB], lnr[MB];
  if constexpr (LN) {
#pragma clang fp contract(off)
    for (int r = wave; r < 16 * MB; r += kSkinnyWaves) {
      const float* xr = g.ln_x + (int64_t)min(r, g.M - 1) * g.ln_ldx;
      float4 v[kLnMaxChunks];
#pragma unroll
      for (int i = 0; i < kLnMaxChunks; ++i) {
        const int c = 4 * (64 * i + lane);
        v[i] = (i < g.ln_nch && c < g.K) ? *(const float4*)(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < kLnMaxChunks; ++i)
        if (i < g.ln_nch) sum += (v[i].x + v[i].y) + (v[i].z + v[i].w);
      const float mean = wave_sum(sum) / (float)g.K;
      float sq = 0.f;
#pragma unroll
      for (int i = 0; i < kLnMaxChunks; ++i) {
        const float a0 = v[i].x - mean, a1 = v[i].y - mean, a2 = v[i].z - mean, a3 = v[i].w - mean;
        if (i < g.ln_nch && (i * 64 + lane) * 4 < g.K) sq += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
      }
      const float inv = rsqrtf(wave_sum(sq) / (float)g.K + g.ln_eps);
      if (lane == 0) {
        ln_mu[r] = mean;
        ln_rs[r] = inv;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      lnm[i] = ln_mu[xrow[i]];
      lnr[i] = ln_rs[xrow[i]];
    }
  }
  // N consecutive normalised X values of row block i from column k
  // (layernorm_kernel's expression per element).
  auto ln_vals = [&](int i, int k, float* out, auto NV) {
#pragma clang fp contract(off)
    constexpr int N = decltype(NV)::value;
    const float* xr = g.ln_x + (int64_t)xrow[i] * g.ln_ldx + k;
#pragma unroll
    for (int h = 0; h < N / 4; ++h) {
      const float4 xv = *(const float4*)(xr + 4 * h);
      const float4 gv = *(const float4*)(g.ln_g + k + 4 * h);
      const float4 bv = *(const float4*)(g.ln_b + k + 4 * h);
      out[4 * h + 0] = (xv.x - lnm[i]) * lnr[i] * gv.x + bv.x;
      out[4 * h + 1] = (xv.y - lnm[i]) * lnr[i] * gv.y + bv.y;
      out[4 * h + 2] = (xv.z - lnm[i]) * lnr[i] * gv.z + bv.z;
      out[4 * h + 3] = (xv.w - lnm[i]) * lnr[i] * gv.w + bv.w;
    }
  };
  auto ln_bf16x8 = [&](int i, int k) {
    float f[8];
    ln_vals(i, k, f, std::integral_constant<int, 8>());
    uint4 u;
    u.x = pack_bf16x2(f[0], f[1]);
    u.y = pack_bf16x2(f[2], f[3]);
    u.z = pack_bf16x2(f[4], f[5]);
    u.w = pack_bf16x2(f[6], f[7]);
    return __builtin_bit_cast(bf16x8_t, u);
  };

  if constexpr (F32) {
    const float* wp = (const float*)g.W + (int64_t)n * g.ldw + kofs + 4 * q;
    const float* xp[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) xp[i] = (const float*)g.X + (int64_t)xrow[i] * g.ldx + kofs + 4 * q;
    // Four k blocks per round: all their loads are issued before the MFMAs.
    auto step = [&](int kb, auto U) {
      constexpr int NU = decltype(U)::value;
      f32x4_t w[NU], x[NU][MB];
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        w[u] = *(const f32x4_t*)(wp + (kb + u) * KB);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          if constexpr (LN) {
            float f[4];
            ln_vals(i, (kb + u) * KB + 4 * q, f, std::integral_constant<int, 4>());
            x[u][i] = f32x4_t{f[0], f[1], f[2], f[3]};
          } else {
            x[u][i] = *(const f32x4_t*)(xp[i] + (kb + u) * KB);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u][i][e], w[u][e], acc[i], 0, 0, 0);
    };
    int kb = kb0;
    for (; kb + 4 <= kb1; kb += 4) step(kb, std::integral_constant<int, 4>());
    for (; kb < kb1; ++kb) step(kb, std::integral_constant<int, 1>());
  } else if constexpr (sizeof(WT) == 1) {
    // fp8: 16 bytes of W per lane and load feed two MFMAs.  Within a 64-wide
    // k step lane quarter q holds k = 16 q + 0..7 for the first MFMA and
    // 16 q + 8..15 for the second, for W and X alike, so every product pairs
    // the same k.
    const uint8_t* wp = (const uint8_t*)g.W + (int64_t)n * g.ldw + kofs + 16 * q;
    const uint16_t* xp[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) xp[i] = (const uint16_t*)g.X + (int64_t)xrow[i] * g.ldx + kofs + 16 * q;
    const int nk2 = g.k_per / 64;
    const int k0 = (nk2 * wave) / kSkinnyWaves, k1 = (nk2 * (wave + 1)) / kSkinnyWaves;
    auto step2 = [&](int kb, auto U) {
      constexpr int NU = decltype(U)::value;
      uint4 wr[NU];
      bf16x8_t x[NU][MB][2];
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        wr[u] = *(const uint4*)(wp + (kb + u) * 64);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          if constexpr (LN) {
            x[u][i][0] = ln_bf16x8(i, (kb + u) * 64 + 16 * q);
            x[u][i][1] = ln_bf16x8(i, (kb + u) * 64 + 16 * q + 8);
          } else {
            x[u][i][0] = *(const bf16x8_t*)(xp[i] + (kb + u) * 64);
            x[u][i][1] = *(const bf16x8_t*)(xp[i] + (kb + u) * 64 + 8);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const bf16x8_t w0 = SkinnyW<uint8_t>::load_pair(wr[u].x, wr[u].y);
        const bf16x8_t w1 = SkinnyW<uint8_t>::load_pair(wr[u].z, wr[u].w);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[u][i][0], w0, acc[i], 0, 0, 0);
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[u][i][1], w1, acc[i], 0, 0, 0);
        }
      }
    };
    int kb = k0;
    for (; kb + 4 <= k1; kb += 4) step2(kb, std::integral_constant<int, 4>());
    for (; kb < k1; ++kb) step2(kb, std::integral_constant<int, 1>());
  } else {
    const WT* wp = (const WT*)g.W + (int64_t)n * g.ldw + kofs + 8 * q;
    const uint16_t* xp[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) xp[i] = (const uint16_t*)g.X + (int64_t)xrow[i] * g.ldx + kofs + 8 * q;
    auto step = [&](int kb, auto U) {
      constexpr int NU = decltype(U)::value;
      bf16x8_t w[NU], x[NU][MB];
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        w[u] = SkinnyW<WT>::load(wp + (kb + u) * KB);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          if constexpr (LN) x[u][i] = ln_bf16x8(i, (kb + u) * KB + 8 * q);
          else x[u][i] = *(const bf16x8_t*)(xp[i] + (kb + u) * KB);
        }
      }
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int i = 0; i < MB; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[u][i], w[u], acc[i], 0, 0, 0);
    };
    int kb = kb0;
    for (; kb + 4 <= kb1; kb += 4) step(kb, std::integral_constant<int, 4>());
    for (; kb < kb1; ++kb) step(kb, std::integral_constant<int, 1>());
  }

  // Sum the 8 waves' partial tiles (fixed order: deterministic).
  __shared__ f32x4_t part[kSkinnyWaves][MB][64];
#pragma unroll
  for (int i = 0; i < MB; ++i) part[wave][i][lane] = acc[i];
  __syncthreads();
  if (wave != 0) return;
  const int col = n0 + c16;
  // At MB = 4 the epilogue inputs are loaded here, after the K loop but still
  // before the first store: a load issued after a store would wait for the
  // store's write acknowledgement too (vmcnt counts both, in order), once per
  // element (config 2's M = 64 MLP down, whose residual is such a load).
  if (!PRE && !g.amax && !g.partial) load_pre();
  const bool ok = col < g.N;
  const float gsc = (g.amax && g.w_scale && ok) ? g.w_scale[col] : 1.f;
  const float gbi = (g.amax && g.bias && ok) ? g.bias[col] : 0.f;
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    f32x4_t v = part[0][i][lane];
#pragma unroll
    for (int w = 1; w < kSkinnyWaves; ++w) v += part[w][i][lane];
    if (g.partial) {
      float* pz = g.partial + (int64_t)blockIdx.y * g.M * g.N;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = i * 16 + 4 * q + e;
        if (row < g.M && ok) pz[(int64_t)row * g.N + col] = v[e];
      }
      continue;
    }
    if (g.amax) {
      // Greedy mode: the row's top-2 over this workgroup's 16 columns (lanes
      // 16 q .. 16 q + 15 hold the same rows), value = sum * scale + bias as
      // epilogue_store_pre computes it.
      const float sc = gsc, bi = gbi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x = v[e];
        if (g.w_scale) x *= sc;
        if (g.bias) x += bi;
        x = nan0_as_inf(x, col);
        float m1 = ok ? x : -INFINITY, m2 = -INFINITY;
        int i1 = ok ? col : 0x7FFFFFFF;
        top2_row16(m1, m2, i1);
        const int row = i * 16 + 4 * q + e;
        if (c16 == 0 && row < g.M)
          g.amax[(int64_t)row * g.amax_ld + blockIdx.x] = make_float4(m1, m2, __int_as_float(i1), 0.f);
      }
      continue;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = i * 16 + 4 * q + e;
      if (row < g.M && col < g.N) epilogue_store_pre(g, row, col, v[e], pre_sc, pre_bi, pre_r[i][e], pre_slot[i][e]);
    }
  }
}

// Greedy-mode reduce: the TPR threads of a row (one wave, or a 256-thread
// workgroup for long rows) fold the row's n_parts top-2 partials (RAW: the
// row's fp32 values themselves) in any order -- the merge keeps the lowest
// index among equal maxima -- and write the index (0 for a row with no
// maximum, as the strict-> scan leaves it) and the top-2 margin.
template <bool RAW, int TPR>
__global__ __launch_bounds__(256) void top2_reduce_kernel(const void* src, int n_parts, int64_t ld, int M,
                                                          int* __restrict__ next, float* __restrict__ margin) {
  constexpr int RPB = 256 / TPR;  // rows per workgroup
  const int t = threadIdx.x % TPR;
  const int row = blockIdx.x * RPB + threadIdx.x / TPR;
  float m1 = -INFINITY, m2 = -INFINITY;
  int i1 = 0x7FFFFFFF;
  if (row < M) {
    if constexpr (RAW) {
      const float* r = (const float*)src + (int64_t)row * ld;
      for (int c = t; c < n_parts; c += TPR) top2_push(m1, m2, i1, nan0_as_inf(r[c], c), c);
    } else {
      const float4* r = (const float4*)src + (int64_t)row * ld;
      for (int c = t; c < n_parts; c += TPR) {
        const float4 p = r[c];
        top2_merge(m1, m2, i1, p.x, p.y, __float_as_int(p.z));
      }
    }
  }
  top2_lanes<64>(m1, m2, i1);
  if constexpr (TPR > 64) {
    __shared__ float s1[TPR / 64], s2[TPR / 64];
    __shared__ int si[TPR / 64];
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { s1[w] = m1; s2[w] = m2; si[w] = i1; }
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int k = 1; k < TPR / 64; ++k) top2_merge(m1, m2, i1, s1[k], s2[k], si[k]);
  } else if (t != 0) {
    return;
  }
  if (row < M) {
    next[row] = i1 == 0x7FFFFFFF ? 0 : i1;
    if (margin) margin[row] = m1 - m2;
  }
}

// Launches the greedy reduce: a wave per row up to 512 partials, else a
// 256-thread workgroup per row (config 5's fp8 lm_head: 16 rows x 2000
// partials, 12.9 -> a few us).
int top2_reduce(bool raw, const void* src, int n_parts, int64_t ld, int M, int* next, float* margin, hipStream_t s) {
  if (n_parts <= 512) {
    const unsigned blocks = (unsigned)cdiv(M, 4);
    if (raw) top2_reduce_kernel<true, 64><<<blocks, 256, 0, s>>>(src, n_parts, ld, M, next, margin);
    else top2_reduce_kernel<false, 64><<<blocks, 256, 0, s>>>(src, n_parts, ld, M, next, margin);
  } else {
    if (raw) top2_reduce_kernel<true, 256><<<(unsigned)M, 256, 0, s>>>(src, n_parts, ld, M, next, margin);
    else top2_reduce_kernel<false, 256><<<(unsigned)M, 256, 0, s>>>(src, n_parts, ld, M, next, margin);
  }
  return check_launch("cbis_gemm_argmax(reduce)");
}

template <typename XT, typename WT, bool LN>
void launch_skinny_mb(const GemmArgs& g, hipStream_t s) {
  const dim3 grid((unsigned)cdiv(g.N, 16), (unsigned)g.ksplit);
  if (g.M <= 16) gemm_skinny_kernel<XT, WT, 1, LN><<<grid, kSkinnyWaves * 64, 0, s>>>(g);
  else if (g.M <= 32) gemm_skinny_kernel<XT, WT, 2, LN><<<grid, kSkinnyWaves * 64, 0, s>>>(g);
  else gemm_skinny_kernel<XT, WT, 4, LN><<<grid, kSkinnyWaves * 64, 0, s>>>(g);
}

template <typename XT, typename WT>
int launch_skinny(const GemmArgs& g, hipStream_t s) {
  if (g.ln_x) launch_skinny_mb<XT, WT, true>(g, s);
  else launch_skinny_mb<XT, WT, false>(g, s);
  return check_launch("cbis_gemm(skinny)");
}

constexpr int kSkinnyMaxM = 64;

// Tile of the bf16 direct-to-LDS path and its split-K plan.  The tile is
// 128 x 128 on 8 waves (2 x 4, each 64 x 32) with a 2-stage 64 KiB ring, so
// two workgroups share a CU.  When the output tiles cannot occupy the 256 CUs
// and K has at least 64 tiles, K is split so about 2 workgroups per CU run;
// each split keeps at least 16 K tiles.  (Measured: at K = 2048 the partial
// round trip costs more than the occupancy gains.)
constexpr int kDmaBM = 128, kDmaBN = 128;
constexpr int kCUs = 256;

struct SplitPlan {
  int ksplit = 1;
  int k_per = 0;
};

// Kernel for a bf16 x bf16 problem on the direct-to-LDS paths, from the
// tile counts (measured on config 4's shapes at M = 1216, TFLOP/s):
//   < kCUs / 2 tiles of 128 x 128, or K < 512: gemm_bf16_dma_kernel, 64 x 64
//     tiles or 128 x 128 with split-K (plan_dma_split); with under 8 K tiles
//     the wave-specialised kernel's ring fill and parked epilogue cost more
//     than they save (config 2, M = 4096, K = 256: 9.5 / 14.1 us against
//     10.8 / 19.1);
//   < kCUs tiles and K of 96 tiles of 64 or more: 160 x 256 tiles with
//     split-K into up to 4 parts, about one workgroup per CU.  With weights
//     cold in HBM, as in the step, this beats whole-K tilings (fc2 at
//     M = 1216: 64 tiles x 4 splits, 62.4 us cold, against 68.2 for
//     split-K 3 on 128 x 128 register-staged and 78.5 for 96 x 128 whole-K;
//     warm, 96 x 128 would be faster);
//   < kCUs tiles otherwise: wave-specialised 96 x 128 (1 x 4 consumers) when
//     its tiles need no more rounds than 128 x 128 ones, else 128 x 128
//     (out-projection: 208 tiles of 96 x 128, 535 TFLOP/s against 466 for
//     160 tiles of 128 x 128);
//   otherwise the wave-specialised tiling with the least estimated time:
//     the busiest CU's tiles (tiles spread over kCUs CUs) times a tile's
//     work, 128 x 256 = 1, 160 x 256 = 1.25, 128 x 128 register-staged = 0.5
//     with a 1.1 penalty for its lower efficiency (two share a CU); ties go
//     to the larger tile.  qkv: 128 x 256 (742 against 645); fc1: 160 x 256, one
//     round of 256 tiles (832 against 685 for 128 x 128 register-staged and
//     577 for 128 x 256); lm_head: 160 x 256 (832 against 779).
enum class Bf16Path { kSmall, kWs128, kWs160Split, kWs96, kWs256, kWs160, kWs128R };

// Split-K parts for 160 x 256 tiles on a deep-K grid: about one workgroup per
// CU, at most 4 parts, each of at least 16 K tiles.
int ws160_splits(int M, int N, int K) {
  const int64_t t160 = cdiv(M, 160) * cdiv(N, 256);
  return (int)std::max<int64_t>(1, std::min<int64_t>({4, kCUs / t160, (K / 64) / 16}));
}

Bf16Path choose_bf16(int M, int N, int K) {
  const int64_t t128 = cdiv(M, 128) * cdiv(N, 128);
  if (t128 < kCUs / 2 || K < 512) return Bf16Path::kSmall;
  if (t128 < kCUs && K / 64 >= 96 && ws160_splits(M, N, K) >= 2) return Bf16Path::kWs160Split;
  if (t128 < kCUs) {
    const double c96 = 0.75 * cdiv(cdiv(M, 96) * cdiv(N, 128), kCUs);
    return c96 < 1.0 ? Bf16Path::kWs96 : Bf16Path::kWs128;
  }
  const double c160 = 1.25 * cdiv(cdiv(M, 160) * cdiv(N, 256), kCUs);
  const double c256 = 1.0 * cdiv(cdiv(M, 128) * cdiv(N, 256), kCUs);
  const double c128 = 0.55 * cdiv(t128, kCUs);
  if (c160 <= c256 && c160 <= c128) return Bf16Path::kWs160;
  if (c256 <= c128) return Bf16Path::kWs256;
  return Bf16Path::kWs128R;
}

SplitPlan plan_dma_split(int M, int N, int K) {
  SplitPlan p;
  p.k_per = K;
  const int64_t tiles = cdiv(M, kDmaBM) * cdiv(N, kDmaBN);
  const int kt = K / 64;
  const Bf16Path path = choose_bf16(M, N, K);
  if (path == Bf16Path::kWs160Split) {
    const int ks = ws160_splits(M, N, K);
    const int per = (kt + ks - 1) / ks;
    p.ksplit = (kt + per - 1) / per;
    p.k_per = per * 64;
    return p;
  }
  if (path != Bf16Path::kSmall || tiles >= kCUs || kt < 64) return p;
  int ks = (int)std::max<int64_t>(2, std::min<int64_t>(4, (2 * kCUs) / tiles));
  ks = std::min(ks, kt / 16);
  if (ks <= 1) return p;
  const int per = (kt + ks - 1) / ks;
  p.ksplit = (kt + per - 1) / per;
  p.k_per = per * 64;
  return p;
}

// Split-K of a skinny call whose reduce runs fused with the LayerNorm after it
// (cbis_gemm_layernorm): when its 16-column workgroups cannot occupy the
// CUs, K is split so the grid reaches up to two workgroups per CU while every
// wave keeps at least two MFMA k steps (config 5's out-projection, K = 2048:
// 2 parts; fc2, K = 8192: 4 parts, the most the fused reduce takes).
SplitPlan plan_skinny_split(int M, int N, int K, int w_dtype) {
  SplitPlan p;
  p.k_per = K;
  const int kstep = w_dtype == CBIS_FP8E4M3 ? 64 : (w_dtype == CBIS_BF16 ? 32 : 16);
  const int64_t wgs = cdiv(N, 16);
  if (M > 64 || wgs >= kCUs) return p;
  for (int ks = 4; ks >= 2; --ks)
    if (wgs * ks <= 2 * kCUs && K % (ks * kstep) == 0 && K / ks >= 2 * kSkinnyWaves * kstep) {
      p.ksplit = ks;
      p.k_per = K / ks;
      break;
    }
  return p;
}

bool dma_eligible(const cbis_gemm_desc* d) {
  return d->x_dtype == CBIS_BF16 && d->w_dtype == CBIS_BF16 && ((uintptr_t)d->W & 15u) == 0 &&
         (d->ldw * 2) % 16 == 0;
}

template <int BM, int BN, int WM, int WN, typename XT, typename WT>
int launch(const GemmArgs& g, hipStream_t s) {
  const int64_t tiles = cdiv(g.M, BM) * cdiv(g.N, BN);
  const size_t lds = std::max(2 * (size_t)(BM + BN) * 128, (size_t)parked_bytes<BM, BN>());
  auto k = gemm_kernel<BM, BN, WM, WN, XT, WT>;
  static bool attr_set = false;  // raise the dynamic-LDS cap once per instantiation
  if (!attr_set && lds > 65536) {
    (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr_set = true;
  }
  k<<<dim3((unsigned)tiles, 1, g.ksplit), WM * WN * 64, lds, s>>>(with_vec(g));
  return check_launch("cbis_gemm");
}

// fp32 x fp32 tiling.  A 32x32x2 fp32 MFMA occupies its SIMD for 64 cycles,
// so one wave per SIMD cannot hide its LDS reads and barriers: large grids
// take 64 x 128 tiles on 8 waves (two per SIMD; config 2 at M = 4096, K =
// 256: QKV 40.9 -> 24.8 us, MLP up 41.4 -> 25.7 against 128 x 128 on 4
// waves), and grids with fewer than 4 workgroups of 4 waves per CU split K
// into up to 4 parts when the caller gives the workspace (config 2, M = 512:
// MLP down 35.5 -> 14.2 us, the K = 256 shapes 13 -> 9.4-11.7 us).
struct F32Plan {
  bool wide;  // 64 x 128 on 8 waves; else 64 x 64 (32 x 64 for M <= 32) on 4 waves
  int ksplit = 1;
  int k_per = 0;
};

F32Plan plan_f32(int M, int N, int K) {
  F32Plan p;
  p.wide = cdiv(M, 128) * cdiv(N, 128) >= 192;
  p.k_per = K;
  if (p.wide) return p;
  const int64_t tiles = M <= 32 ? cdiv(M, 32) * cdiv(N, 64) : cdiv(M, 64) * cdiv(N, 64);
  const int kt = K / 32;
  // A grid that already gives every CU a workgroup splits only deep K (each
  // part >= 8 K tiles): config 2's out-projection at M = 4096 (256 tiles,
  // K = 256) measured 13.5 us whole and 17.3 in two parts.
  const int min_kt = tiles >= kCUs ? 8 : 4;
  const int ks = (int)std::min<int64_t>({4, (4 * kCUs) / std::max<int64_t>(1, tiles), kt / min_kt});
  if (ks <= 1) return p;
  const int per = (kt + ks - 1) / ks;
  p.ksplit = (kt + per - 1) / per;
  p.k_per = per * 32;
  return p;
}

// Picks a tile shape from the problem size: the largest tile that still
// gives the 256 CUs at least about one workgroup each.
template <typename XT, typename WT>
int dispatch(const GemmArgs& g, hipStream_t s) {
  const int64_t t128 = cdiv(g.M, 128) * cdiv(g.N, 128);
  if constexpr (sizeof(XT) == 4) {
    if (plan_f32(g.M, g.N, g.K).wide) return launch<64, 128, 2, 4, XT, WT>(g, s);
    if (g.M <= 32) return launch<32, 64, 1, 2, XT, WT>(g, s);
    return launch<64, 64, 2, 2, XT, WT>(g, s);
  } else {
    if (t128 >= 192) return launch<128, 128, 2, 2, XT, WT>(g, s);
    if (g.M <= 32) return launch<32, 128, 1, 4, XT, WT>(g, s);
    return launch<64, 128, 2, 2, XT, WT>(g, s);
  }
}

// Column-tile width of the greedy-mode partials for d's GEMM path: the
// kernels that reduce in their epilogue are the skinny one (16 columns per
// workgroup) and the wave-specialised bf16 ones (their BN); 0 for the others
// (fp32 or fp8 weights at M > 64, small bf16 grids), whose logits
// cbis_gemm_argmax stores and reduces instead.  Follows gemm_run's choice.
int argmax_tile_cols(const cbis_gemm_desc* d) {
  const int we = d->w_dtype == CBIS_F32 ? 4 : (d->w_dtype == CBIS_BF16 ? 2 : 1);
  const bool w_al = ((uintptr_t)d->W & 15u) == 0 && (d->ldw * we) % 16 == 0;
  if (d->M <= kSkinnyMaxM && w_al && d->K % (d->w_dtype == CBIS_FP8E4M3 ? 64 : 32) == 0) return 16;
  if (d->x_dtype != CBIS_BF16 || d->w_dtype != CBIS_BF16 || !dma_eligible(d)) return 0;
  switch (choose_bf16(d->M, d->N, d->K)) {
    case Bf16Path::kWs256:
    case Bf16Path::kWs160: return 256;
    case Bf16Path::kWs128:
    case Bf16Path::kWs96:
    case Bf16Path::kWs160Split:  // unsplit in greedy mode: 96 x 128 tiles
    case Bf16Path::kWs128R: return 128;
    case Bf16Path::kSmall: break;
  }
  return 0;
}

// Validates the descriptor and launches the product kernel (no split-K
// reduce); g receives the arguments it ran with (g.ksplit > 1: the raw sums
// are in the workspace partials and still need their reduce).  With amax the
// kernel runs in greedy mode (no Y; never split): the caller checked that
// argmax_tile_cols(d) > 0 and sized amax [M][cdiv(N, that)].
// LayerNorm prologue arguments of cbis_layernorm_gemm.
struct LnPrologue {
  const float* x;
  int64_t ldx;
  const float* gamma;
  const float* beta;
  float eps;
};

// Whether d's GEMM runs on the skinny (decode-sized) kernel.
bool skinny_path(const cbis_gemm_desc* d) {
  const int we = d->w_dtype == CBIS_F32 ? 4 : (d->w_dtype == CBIS_BF16 ? 2 : 1);
  const bool w_al = ((uintptr_t)d->W & 15u) == 0 && (d->ldw * we) % 16 == 0;
  return d->M <= kSkinnyMaxM && w_al && d->K % (d->w_dtype == CBIS_FP8E4M3 ? 64 : 32) == 0;
}

// Whether a plain call (no greedy epilogue, LayerNorm prologue or fused
// split-K reduce, which are the skinny kernel's own) of decode-sized M runs
// on the skinny kernel: always up to 32 rows; bf16 x bf16 calls of 33..64
// rows take the direct-to-LDS tiles instead, whose workgroups read X once
// per tile where the skinny kernel reads all of it once per 16 columns
// (config 2 at M = 64, qkv / out / MLP up / MLP down: 7.0 / 7.0 / 7.6 / 10.4
// us skinny, 4.2 / 4.2 / 4.7 / 7.0 tiled).  fp32 weights keep the skinny
// kernel (M = 64 qkv 8.3 us against 9.1 on the fp32 tiles), fp8 weights too.
bool plain_skinny(const cbis_gemm_desc* d) {
  return skinny_path(d) && (d->M <= 32 || !dma_eligible(d));
}

// Whether cbis_layernorm_gemm(_argmax) forms d's LayerNorm inside the GEMM.
bool ln_prologue_ok(const cbis_gemm_desc* d, const float* x, int64_t ldx, const float* gamma, const float* beta) {
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  return skinny_path(d) && d->K % 4 == 0 && d->K <= kLnPrologueMaxK && a16(x) && ldx % 4 == 0 && a16(gamma) &&
         a16(beta);
}

// fused_reduce: the caller folds split-K partials into the kernel that runs
// next (cbis_gemm_layernorm), so a skinny call may split too.
int gemm_run(const cbis_gemm_desc* d, hipStream_t s, GemmArgs& g, float4* amax = nullptr,
             const LnPrologue* ln = nullptr, bool fused_reduce = false) {
  g.ksplit = 1;
  CBIS_REQUIRE(d, CBIS_ERR_INVALID, "cbis_gemm: null descriptor");
  CBIS_REQUIRE(d->M >= 0 && d->N > 0 && d->K > 0, CBIS_ERR_INVALID, "cbis_gemm: bad M/N/K %d/%d/%d", d->M, d->N, d->K);
  if (d->M == 0) return CBIS_OK;
  CBIS_REQUIRE(d->X && d->W, CBIS_ERR_INVALID, "cbis_gemm: null X/W");
  const bool f32 = d->x_dtype == CBIS_F32;
  CBIS_REQUIRE((f32 && d->w_dtype == CBIS_F32) ||
                   (d->x_dtype == CBIS_BF16 && (d->w_dtype == CBIS_BF16 || d->w_dtype == CBIS_FP8E4M3)),
               CBIS_ERR_UNSUPPORTED, "cbis_gemm: x dtype %d with w dtype %d", d->x_dtype, d->w_dtype);
  const int bk = f32 ? 32 : 64;
  CBIS_REQUIRE(d->K % bk == 0, CBIS_ERR_UNSUPPORTED, "cbis_gemm: K=%d must be a multiple of %d", d->K, bk);
  const int xe = f32 ? 4 : 2;
  const int we = d->w_dtype == CBIS_F32 ? 4 : (d->w_dtype == CBIS_BF16 ? 2 : 1);
  CBIS_REQUIRE(((uintptr_t)d->X & 15u) == 0 && (d->ldx * xe) % 16 == 0 && d->ldx >= d->K, CBIS_ERR_INVALID,
               "cbis_gemm: X rows must be 16-byte aligned");
  CBIS_REQUIRE(((uintptr_t)d->W & 7u) == 0 && (d->ldw * we) % 8 == 0 && d->ldw >= d->K, CBIS_ERR_INVALID,
               "cbis_gemm: W rows must be 8-byte aligned");
  CBIS_REQUIRE(d->w_dtype != CBIS_FP8E4M3 || d->w_scale, CBIS_ERR_INVALID, "cbis_gemm: fp8 weights need w_scale");
  CBIS_REQUIRE(d->y_dtype == CBIS_F32 || d->y_dtype == CBIS_BF16, CBIS_ERR_UNSUPPORTED, "cbis_gemm: y dtype");
  CBIS_REQUIRE(d->epilogue == CBIS_EPI_NONE || d->epilogue == CBIS_EPI_GELU, CBIS_ERR_INVALID, "cbis_gemm: epilogue");
  const bool kv = d->k_pool != nullptr;
  if (kv) {
    CBIS_REQUIRE(d->v_pool && d->write_page && d->write_offset && d->kv_width > 0 && d->page_size > 0 &&
                     d->kv_col0 >= 0 && d->kv_col0 + 2 * d->kv_width == d->N,
                 CBIS_ERR_INVALID, "cbis_gemm: K/V scatter needs kv_col0 + 2*kv_width == N and slot arrays");
    CBIS_REQUIRE(d->kv_dtype == CBIS_F32 || d->kv_dtype == CBIS_BF16, CBIS_ERR_UNSUPPORTED, "cbis_gemm: kv dtype");
  }
  // Y may be absent only in greedy mode or when every column goes to the K/V pages.
  CBIS_REQUIRE(amax || (kv && d->kv_col0 == 0) || d->Y, CBIS_ERR_INVALID, "cbis_gemm: null Y");

  g.M = d->M; g.N = d->N; g.K = d->K;
  g.n_fast = (int64_t)d->M * xe > (int64_t)d->N * we ? 1 : 0;
  g.X = d->X; g.ldx = d->ldx;
  g.W = d->W; g.ldw = d->ldw;
  g.w_scale = d->w_scale;
  g.bias = d->bias;
  g.gelu = d->epilogue == CBIS_EPI_GELU;
  g.residual = d->residual; g.ldr = d->ldr;
  g.y_bf16 = d->y_dtype == CBIS_BF16;
  g.Y = d->Y; g.ldy = d->ldy;
  g.kv_col0 = kv ? d->kv_col0 : 0x7FFFFFFF;
  g.kv_width = d->kv_width; g.kv_bf16 = d->kv_dtype == CBIS_BF16; g.page_size = d->page_size;
  g.k_pool = kv ? d->k_pool : nullptr; g.v_pool = d->v_pool;
  g.wpage = d->write_page; g.woff = d->write_offset;
  g.ksplit = 1;
  g.k_per = d->K;
  g.partial = nullptr;
  g.amax = amax;
  g.amax_ld = amax ? (int)cdiv(d->N, argmax_tile_cols(d)) : 0;
  g.ln_x = ln ? ln->x : nullptr;
  g.ln_ldx = ln ? ln->ldx : 0;
  g.ln_g = ln ? ln->gamma : nullptr;
  g.ln_b = ln ? ln->beta : nullptr;
  g.ln_eps = ln ? ln->eps : 0.f;
  g.ln_nch = ln ? ln_chunks(d->K) : 0;
  CBIS_REQUIRE(!ln || skinny_path(d), CBIS_ERR_UNSUPPORTED, "cbis_layernorm_gemm: LayerNorm prologue off the skinny path");

  // Decode-sized M: weight streaming (K a multiple of 32 for bf16 and fp32,
  // of 64 for fp8; W rows 16-byte aligned).
  if (amax || ln || fused_reduce ? skinny_path(d) : plain_skinny(d)) {
    if (fused_reduce && !amax && !ln) {
      const SplitPlan p = plan_skinny_split(d->M, d->N, d->K, d->w_dtype);
      const size_t need = (size_t)p.ksplit * d->M * d->N * sizeof(float);
      if (p.ksplit > 1 && d->workspace && d->workspace_bytes >= need && ((uintptr_t)d->workspace & 15u) == 0) {
        g.ksplit = p.ksplit;
        g.k_per = p.k_per;
        g.partial = (float*)d->workspace;
      }
    }
    if (f32) return launch_skinny<float, float>(g, s);
    if (d->w_dtype == CBIS_BF16) return launch_skinny<uint16_t, uint16_t>(g, s);
    return launch_skinny<uint16_t, uint8_t>(g, s);
  }
  if (f32) {
    const F32Plan p = plan_f32(d->M, d->N, d->K);
    const size_t need = (size_t)p.ksplit * d->M * d->N * sizeof(float);
    if (!amax && p.ksplit > 1 && d->workspace && d->workspace_bytes >= need) {
      g.ksplit = p.ksplit;
      g.k_per = p.k_per;
      g.partial = (float*)d->workspace;
    }
    return dispatch<float, float>(g, s);
  }
  if (d->w_dtype == CBIS_BF16) {
    // The direct-to-LDS path needs 16-byte aligned rows of both operands.
    if (dma_eligible(d)) {
      const Bf16Path path = choose_bf16(d->M, d->N, d->K);
      const SplitPlan p = plan_dma_split(d->M, d->N, d->K);
      const size_t need = (size_t)p.ksplit * d->M * d->N * sizeof(float);
      const bool split = !amax && p.ksplit > 1 && d->workspace && d->workspace_bytes >= need;
      if (split) {
        g.ksplit = p.ksplit;
        g.k_per = p.k_per;
        g.partial = (float*)d->workspace;
      }
      switch (path) {
        case Bf16Path::kWs256: return launch_ws<128, 256, 3>(g, s);
        case Bf16Path::kWs160: return launch_ws<160, 256, 3, 0, 1>(g, s);
        case Bf16Path::kWs128: return launch_ws<128, 128, 3>(g, s);
        case Bf16Path::kWs96: return launch_ws<96, 128, 3, 0, 1>(g, s);
        case Bf16Path::kWs160Split:
          return split ? launch_ws<160, 256, 3, 0, 1>(g, s) : launch_ws<96, 128, 3, 0, 1>(g, s);
        case Bf16Path::kWs128R: return launch_ws<128, 128, 2, 3>(g, s);
        case Bf16Path::kSmall: break;
      }
      // Grids with fewer 128 x 128 tiles than CUs run 64 x 64 tiles (4 waves
      // of 32 x 32): four times the workgroups (config 4's out-projection,
      // 160 tiles: 28.3 -> 23.4 us).  A third ring slot pays when the grid
      // fills the CUs and K has 8 or more tiles (config 2's MLP down at
      // M = 4096, K = 1024: 12.2 -> 10.7 us; at M = 512 it costs 1 us).
      if (g.ksplit == 1 && cdiv(d->M, kDmaBM) * cdiv(d->N, kDmaBN) < kCUs) {
        if (d->K >= 512 && cdiv(d->M, 64) * cdiv(d->N, 64) >= kCUs) return launch_dma<64, 64, 2, 2, 3>(g, s);
        return launch_dma<64, 64, 2, 2, 2>(g, s);
      }
      return launch_dma<kDmaBM, kDmaBN, 2, 4, 2>(g, s);
    }
    return dispatch<uint16_t, uint16_t>(g, s);
  }
  return dispatch<uint16_t, uint8_t>(g, s);
}

int gemm_argmax(const cbis_gemm_desc* d, int* next_token, float* margin, void* workspace, size_t workspace_bytes,
                hipStream_t s, const LnPrologue* ln, const char* who) {
  CBIS_REQUIRE(d, CBIS_ERR_INVALID, "%s: null descriptor", who);
  CBIS_REQUIRE(d->epilogue == CBIS_EPI_NONE && !d->residual && !d->k_pool, CBIS_ERR_INVALID,
               "%s: the greedy epilogue takes the scale and bias only (no GELU, residual or K/V scatter)", who);
  CBIS_REQUIRE(next_token, CBIS_ERR_INVALID, "%s: null next_token", who);
  if (d->M == 0) return CBIS_OK;
  const size_t need = cbis_gemm_argmax_workspace_size(d);
  CBIS_REQUIRE(workspace && workspace_bytes >= need && ((uintptr_t)workspace & 15u) == 0, CBIS_ERR_WORKSPACE,
               "%s: workspace %zu bytes (16-byte aligned), need %zu", who, workspace_bytes, need);
  const int cols = argmax_tile_cols(d);
  if (cols > 0) {
    GemmArgs g;
    const int rc = gemm_run(d, s, g, (float4*)workspace, ln);
    if (rc) return rc;
    return top2_reduce(false, workspace, g.amax_ld, g.amax_ld, d->M, next_token, margin, s);
  }
  // Paths without a greedy epilogue: the logits into d->Y (when it is an fp32
  // [M, N] buffer) or the workspace, then the same reduce over them.
  cbis_gemm_desc e = *d;
  const bool y_given = d->Y && d->y_dtype == CBIS_F32 && d->ldy >= d->N;
  const size_t lg = y_given ? 0 : (size_t)d->M * d->N * sizeof(float);
  if (!y_given) {
    e.y_dtype = CBIS_F32;
    e.Y = workspace;
    e.ldy = d->N;
  }
  e.workspace = (char*)workspace + lg;
  e.workspace_bytes = workspace_bytes - lg;
  CBIS_REQUIRE(!ln, CBIS_ERR_UNSUPPORTED, "%s: LayerNorm prologue on a path that stores logits", who);
  const int rc = cbis_gemm(&e, (cbis_stream_t)s);
  if (rc) return rc;
  return top2_reduce(true, e.Y, d->N, e.ldy, d->M, next_token, margin, s);
}


int splitk_reduce(const GemmArgs& g, hipStream_t s) {
  splitk_reduce_kernel<<<splitk_reduce_blocks(g), 256, 0, s>>>(g);
  return check_launch("cbis_gemm(split-k reduce)");
}
}  // namespace
}  // namespace cbis

using namespace cbis;

extern "C" {

int cbis_gemm(const cbis_gemm_desc* d, cbis_stream_t stream) {
  hipStream_t s = (hipStream_t)stream;
  GemmArgs g;
  const int rc = gemm_run(d, s, g);
  if (rc || g.ksplit <= 1) return rc;
  return splitk_reduce(g, s);
}

int cbis_gemm_layernorm(const cbis_gemm_desc* d, const float* ln_gamma, const float* ln_beta, float eps, int ln_dtype,
                        void* ln_out, int64_t ld_ln, cbis_stream_t stream) {
  CBIS_REQUIRE(d, CBIS_ERR_INVALID, "cbis_gemm_layernorm: null descriptor");
  CBIS_REQUIRE(d->y_dtype == CBIS_F32 && d->k_pool == nullptr && d->Y, CBIS_ERR_INVALID,
               "cbis_gemm_layernorm: needs an fp32 Y and no K/V scatter");
  CBIS_REQUIRE(d->N % 4 == 0 && d->N <= 8192, CBIS_ERR_UNSUPPORTED,
               "cbis_gemm_layernorm: row length %d (needs a multiple of 4, <= 8192)", d->N);
  CBIS_REQUIRE(ln_gamma && ln_beta && ln_out, CBIS_ERR_INVALID, "cbis_gemm_layernorm: null LayerNorm pointer");
  CBIS_REQUIRE(ln_dtype == CBIS_F32 || ln_dtype == CBIS_BF16, CBIS_ERR_UNSUPPORTED, "cbis_gemm_layernorm: ln dtype");
  CBIS_REQUIRE(ld_ln % 4 == 0 && ((uintptr_t)ln_out & (ln_dtype == CBIS_F32 ? 15u : 7u)) == 0 && d->ldy % 4 == 0 &&
                   ((uintptr_t)d->Y & 15u) == 0,
               CBIS_ERR_INVALID, "cbis_gemm_layernorm: misaligned rows");
  hipStream_t s = (hipStream_t)stream;
  GemmArgs g;
  int rc = gemm_run(d, s, g, nullptr, nullptr, true);
  if (rc || d->M == 0) return rc;
  // layernorm_kernel's chunk count for this row length (its VPL).
  const int nch = ln_chunks(d->N);
  const int vpw = (nch + 3) / 4;
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const bool fuse = g.ksplit > 1 && g.ksplit <= 4 && vpw <= 4 && !g.gelu && a16(g.partial) &&
                    (!g.w_scale || a16(g.w_scale)) && (!g.bias || a16(g.bias)) &&
                    (!g.residual || (a16(g.residual) && g.ldr % 4 == 0)) && a16(ln_gamma) && a16(ln_beta);
  if (!fuse) {
    if (g.ksplit > 1 && (rc = splitk_reduce(g, s))) return rc;
    return cbis_layernorm(d->M, d->N, (const float*)d->Y, d->ldy, ln_gamma, ln_beta, eps, ln_dtype, ln_out, ld_ln,
                          stream);
  }
  const dim3 grid((unsigned)d->M);
#define CBIS_SKLN(V, KS)                                                                                      \
  if (ln_dtype == CBIS_F32)                                                                                   \
    splitk_layernorm_kernel<V, KS, float><<<grid, 256, 0, s>>>(g, ln_gamma, ln_beta, eps, nch, (float*)ln_out, \
                                                                ld_ln);                                       \
  else                                                                                                        \
    splitk_layernorm_kernel<V, KS, uint16_t><<<grid, 256, 0, s>>>(g, ln_gamma, ln_beta, eps, nch,              \
                                                                   (uint16_t*)ln_out, ld_ln);
#define CBIS_SKLN_KS(V)                      \
  if (g.ksplit == 2) { CBIS_SKLN(V, 2) }     \
  else if (g.ksplit == 3) { CBIS_SKLN(V, 3) } \
  else { CBIS_SKLN(V, 4) }
  if (vpw <= 1) { CBIS_SKLN_KS(1) }
  else if (vpw <= 2) { CBIS_SKLN_KS(2) }
  else { CBIS_SKLN_KS(4) }
#undef CBIS_SKLN_KS
#undef CBIS_SKLN
  return check_launch("cbis_gemm_layernorm(split-k reduce + layernorm)");
}

int cbis_layernorm_gemm(const cbis_gemm_desc* d, const float* x, int64_t ldx, const float* ln_gamma,
                        const float* ln_beta, float eps, cbis_stream_t stream) {
  const char* who = "cbis_layernorm_gemm";
  CBIS_REQUIRE(d, CBIS_ERR_INVALID, "%s: null descriptor", who);
  CBIS_REQUIRE(x && ln_gamma && ln_beta && d->X, CBIS_ERR_INVALID, "%s: null x / LayerNorm / X pointer", who);
  CBIS_REQUIRE(d->x_dtype == CBIS_F32 || d->x_dtype == CBIS_BF16, CBIS_ERR_UNSUPPORTED, "%s: x dtype", who);
  CBIS_REQUIRE(ldx >= d->K, CBIS_ERR_INVALID, "%s: ldx %lld < K %d", who, (long long)ldx, d->K);
  if (d->M == 0) return CBIS_OK;
  if (!ln_prologue_ok(d, x, ldx, ln_gamma, ln_beta)) {
    const int rc = cbis_layernorm(d->M, d->K, x, ldx, ln_gamma, ln_beta, eps, d->x_dtype, (void*)d->X, d->ldx, stream);
    if (rc) return rc;
    return cbis_gemm(d, stream);
  }
  hipStream_t s = (hipStream_t)stream;
  GemmArgs g;
  const LnPrologue ln = {x, ldx, ln_gamma, ln_beta, eps};
  return gemm_run(d, s, g, nullptr, &ln);
}

size_t cbis_gemm_argmax_workspace_size(const cbis_gemm_desc* d) {
  if (!d || d->M <= 0 || d->N <= 0 || d->K <= 0) return 0;
  const int cols = argmax_tile_cols(d);
  if (cols > 0) return (size_t)d->M * cdiv(d->N, cols) * sizeof(float4);
  // The logits (unless d->Y takes them) and the split-K partials.
  const bool y_given = d->Y && d->y_dtype == CBIS_F32 && d->ldy >= d->N;
  return (y_given ? 0 : (size_t)d->M * d->N * sizeof(float)) + cbis_gemm_workspace_size(d);
}

int cbis_gemm_argmax(const cbis_gemm_desc* d, int* next_token, float* margin, void* workspace,
                     size_t workspace_bytes, cbis_stream_t stream) {
  return gemm_argmax(d, next_token, margin, workspace, workspace_bytes, (hipStream_t)stream, nullptr,
                     "cbis_gemm_argmax");
}

int cbis_layernorm_gemm_argmax(const cbis_gemm_desc* d, const float* x, int64_t ldx, const float* ln_gamma,
                               const float* ln_beta, float eps, int* next_token, float* margin, void* workspace,
                               size_t workspace_bytes, cbis_stream_t stream) {
  const char* who = "cbis_layernorm_gemm_argmax";
  CBIS_REQUIRE(d, CBIS_ERR_INVALID, "%s: null descriptor", who);
  CBIS_REQUIRE(x && ln_gamma && ln_beta && d->X, CBIS_ERR_INVALID, "%s: null x / LayerNorm / X pointer", who);
  CBIS_REQUIRE(d->x_dtype == CBIS_F32 || d->x_dtype == CBIS_BF16, CBIS_ERR_UNSUPPORTED, "%s: x dtype", who);
  CBIS_REQUIRE(ldx >= d->K, CBIS_ERR_INVALID, "%s: ldx %lld < K %d", who, (long long)ldx, d->K);
  if (d->M == 0) return CBIS_OK;
  if (!ln_prologue_ok(d, x, ldx, ln_gamma, ln_beta)) {
    const int rc = cbis_layernorm(d->M, d->K, x, ldx, ln_gamma, ln_beta, eps, d->x_dtype, (void*)d->X, d->ldx, stream);
    if (rc) return rc;
    return cbis_gemm_argmax(d, next_token, margin, workspace, workspace_bytes, stream);
  }
  const LnPrologue ln = {x, ldx, ln_gamma, ln_beta, eps};
  return gemm_argmax(d, next_token, margin, workspace, workspace_bytes, (hipStream_t)stream, &ln, who);
}

size_t cbis_gemm_layernorm_workspace_size(const cbis_gemm_desc* d) {
  if (!d || d->M <= 0 || d->N <= 0 || d->K <= 0) return 0;
  // Skinny calls split only here, where the LayerNorm kernel folds the
  // partials in (plan_skinny_split).
  const int we = d->w_dtype == CBIS_F32 ? 4 : (d->w_dtype == CBIS_BF16 ? 2 : 1);
  if (d->M <= kSkinnyMaxM && ((uintptr_t)d->W & 15u) == 0 && (d->ldw * we) % 16 == 0 &&
      d->K % (d->w_dtype == CBIS_FP8E4M3 ? 64 : 32) == 0) {
    const SplitPlan p = plan_skinny_split(d->M, d->N, d->K, d->w_dtype);
    return p.ksplit > 1 ? (size_t)p.ksplit * d->M * d->N * sizeof(float) : 0;
  }
  return cbis_gemm_workspace_size(d);
}

size_t cbis_gemm_workspace_size(const cbis_gemm_desc* d) {
  if (!d || d->M <= 0 || d->N <= 0 || d->K <= 0) return 0;
  // gemm_run's skinny path never splits in cbis_gemm.
  if (plain_skinny(d)) return 0;
  if (d->x_dtype == CBIS_F32 && d->w_dtype == CBIS_F32) {
    // gemm_run's fp32 paths: the skinny kernel (no split) or plan_f32.
    const bool w_al = ((uintptr_t)d->W & 15u) == 0 && (d->ldw * 4) % 16 == 0;
    if ((d->M <= kSkinnyMaxM && w_al && d->K % 32 == 0) || d->K % 32) return 0;
    const F32Plan p = plan_f32(d->M, d->N, d->K);
    return p.ksplit > 1 ? (size_t)p.ksplit * d->M * d->N * sizeof(float) : 0;
  }
  if (!dma_eligible(d) || d->K % 64) return 0;
  const SplitPlan p = plan_dma_split(d->M, d->N, d->K);
  return p.ksplit > 1 ? (size_t)p.ksplit * d->M * d->N * sizeof(float) : 0;
}

int cbis_linear_forward(const float* X, const float* W, const float* b, float* Y, int T, int in_features,
                        int out_features, cbis_stream_t stream) {
  cbis_gemm_desc d = {};
  d.M = T; d.N = out_features; d.K = in_features;
  d.x_dtype = CBIS_F32; d.X = X; d.ldx = in_features;
  d.w_dtype = CBIS_F32; d.W = W; d.ldw = in_features;
  d.bias = b;
  d.y_dtype = CBIS_F32; d.Y = Y; d.ldy = out_features;
  return cbis_gemm(&d, stream);
}

}  // extern "C"
