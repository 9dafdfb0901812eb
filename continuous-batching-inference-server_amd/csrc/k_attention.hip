// Paged causal attention for gfx950.
//
// Reference: fused_attention_kernel, kernels/attention.cu:57-98 -- one 32-lane
// warp per (row, head) walking keys one at a time (page lookup, shuffle-tree
// dot, two expf per key).  Semantics kept: row r attends to keys
// j in [0, pos_r] of its sequence (kv_len = pos_r + 1, :67-68), key j is slot
// j % page_size of physical page table[j / page_size] (:79-83), scores are
// scaled by 1/sqrt(head_dim) (:72) and softmax-normalised (python/model.py:40-44).
//
// Decode kernel (HBM-bound).  A workgroup of NW = 8 waves (16 for launches
// of at least one workgroup per CU in one pass, or two per CU in splits)
// owns one (row, head block, kv split).  A head block is the heads whose head_dim
// slices of one token row form 1 KiB: 8 heads for fp32 K/V, 16 for bf16 (the
// last block of a head count that is not a multiple is partial), so
// one 16-byte-per-lane wave load reads one token's slice of the block fully
// coalesced, and a 16-token page is 16 such loads at the token stride.  Each
// lane holds 4 (fp32) or 8 (bf16) dims of one head; q.k is finished with
// 2-3 DPP steps inside the lane group.  Waves take whole pages round-robin,
// run an online softmax per page (one max / rescale per 16 keys, exp2 with
// log2(e) folded into q), merge through LDS, and either write the output
// (single split) or fp32 partials (m, l, acc) that a merge kernel combines.
//
// Prefill kernel (MFMA).  One workgroup per (query tile of up to 64 rows,
// head pair); a head's two waves take the key blocks round-robin and merge at
// the end.  S^T = K Q^T on v_mfma_f32_32x32x16_bf16 with K read straight
// from the pages in the A-operand layout, online softmax per query column,
// O^T = V^T P^T with P taken from the S^T accumulators in registers (their
// lane layout is the B-operand layout up to a fixed permutation of the key
// index, applied to V^T as well) and V^T read from an LDS copy of the 32-key
// V tile with gfx950's transposing LDS read (ds_read_b64_tr_b16).
#include <mutex>
#include <type_traits>

#include "common.hpp"

namespace cbis {
namespace {

constexpr int kHD = 32;  // head_dim supported by these kernels
constexpr int kPS = 16;  // page_size supported by these kernels
constexpr int kWS = kHD + 4;  // floats per split partial: acc[32], m, l, pad
constexpr int kResidentWaves = 256 * 32;  // decode waves resident on the 256 CUs (64 VGPRs each)

struct DecodeArgs {
  const int* rows;
  const void* q;
  int64_t ldq;
  int q_bf16;
  const void* kpool;
  const void* vpool;
  int num_pages;
  const int* bt;
  int64_t bt_stride;
  const int* row_bt;
  const int* row_pos;
  void* out;
  int64_t ldo;
  int out_bf16;
  float* ws;  // [n_rows][n_splits][H][kWS]: acc[kHD], m, l, 2 pad (16-byte rows)
  int n_heads;
  int n_hblocks;
  int n_splits;
  int split_tokens;
  int max_kv;  // clamp for kv_len (bt_stride * page_size)
  float qscale;
  // The out-projection of cbis_paged_attention_proj (read only by the
  // paged_decode_kernel instantiations with a weight type): Y[row, n] =
  // attn(row) . W[n, :] (* scale[n]) (+ bias[n]) (+ res[row, n]) for the
  // workgroup's 64 columns n; the grid is p_rows x (D / 64) workgroups.
  const void* pw;
  int64_t pldw;
  const float* pscale;
  const float* pbias;
  const float* pres;
  int64_t pldr;
  float* py;
  int64_t pldy;
  int p_rows;
  int pkpt;     // k per thread: D / 8
  int px_bf16;  // the attention output is rounded to bf16 before the product
};

template <typename KVT>
struct KVTraits;
template <>
struct KVTraits<float> {
  static constexpr int EPL = 4;  // elements per 16-byte lane load
  __device__ static inline void unpack(const uint4& r, float* f) {
    f[0] = __uint_as_float(r.x);
    f[1] = __uint_as_float(r.y);
    f[2] = __uint_as_float(r.z);
    f[3] = __uint_as_float(r.w);
  }
};
template <>
struct KVTraits<uint16_t> {
  static constexpr int EPL = 8;
  __device__ static inline void unpack(const uint4& r, float* f) {
    f[0] = bf16lo(r.x); f[1] = bf16hi(r.x);
    f[2] = bf16lo(r.y); f[3] = bf16hi(r.y);
    f[4] = bf16lo(r.z); f[5] = bf16hi(r.z);
    f[6] = bf16lo(r.w); f[7] = bf16hi(r.w);
  }
};

// K/V pages are read once per step: non-temporal loads stream them past the
// caches (on MI355X a streaming read reaches ~7.1 TB/s this way against
// ~6.2 TB/s with ordinary loads).
template <typename T>
__device__ inline uint4 load_stream(const T* p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// A fused workgroup's share of the out-projection weights: thread t takes
// column part * 64 + (t >> 3) and k = (t & 7) * kpt .. + kpt - 1 (kpt <= KMAX),
// loaded when the kernel starts, so their round trip overlaps the attention's.
template <typename WT>
struct ProjW {
  __device__ void load(const DecodeArgs&, int, int) {}
};
template <>
struct ProjW<float> {
  static constexpr int KMAX = 32;
  float4 w[KMAX / 4];
  __device__ void load(const DecodeArgs& a, int part, int t) {
    const float* p = (const float*)a.pw + (int64_t)(part * 64 + (t >> 3)) * a.pldw + (t & 7) * a.pkpt;
#pragma unroll
    for (int i = 0; i < KMAX / 4; ++i)
      if (4 * i < a.pkpt) w[i] = *(const float4*)(p + 4 * i);
  }
  // sum over this thread's k of x[k] * W[n, k], in k order
  __device__ float dot(const DecodeArgs& a, const float* x) const {
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < KMAX / 4; ++i) {
      if (4 * i >= a.pkpt) break;
      const float4 v = *(const float4*)(x + 4 * i);
      d += v.x * w[i].x;
      d += v.y * w[i].y;
      d += v.z * w[i].z;
      d += v.w * w[i].w;
    }
    return d;
  }
};
template <>
struct ProjW<uint16_t> {  // bf16
  static constexpr int KMAX = 64;
  uint4 w[KMAX / 8];
  __device__ void load(const DecodeArgs& a, int part, int t) {
    const uint16_t* p = (const uint16_t*)a.pw + (int64_t)(part * 64 + (t >> 3)) * a.pldw + (t & 7) * a.pkpt;
#pragma unroll
    for (int i = 0; i < KMAX / 8; ++i)
      if (8 * i < a.pkpt) w[i] = *(const uint4*)(p + 8 * i);
  }
  __device__ float dot(const DecodeArgs& a, const float* x) const {
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < KMAX / 8; ++i) {
      if (8 * i >= a.pkpt) break;
      const float4 v0 = *(const float4*)(x + 8 * i), v1 = *(const float4*)(x + 8 * i + 4);
      d += v0.x * bf16lo(w[i].x);
      d += v0.y * bf16hi(w[i].x);
      d += v0.z * bf16lo(w[i].y);
      d += v0.w * bf16hi(w[i].y);
      d += v1.x * bf16lo(w[i].z);
      d += v1.y * bf16hi(w[i].z);
      d += v1.z * bf16lo(w[i].w);
      d += v1.w * bf16hi(w[i].w);
    }
    return d;
  }
};

// WT void: decode attention.  WT float / uint16_t (bf16): the same
// attention for one-pass rows of one head block, each row's workgroups then
// applying the out-projection to it (cbis_paged_attention_proj).
template <typename KVT, int NW, typename WT = void>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(const DecodeArgs a) {
  constexpr bool PROJ = !std::is_void<WT>::value;
  constexpr int EPL = KVTraits<KVT>::EPL;
  constexpr int G = kHD / EPL;  // lanes per head
  constexpr int HPB = 64 / G;   // heads per block (one 1 KiB wave load)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  int bid = blockIdx.x;
  int part = 0;
  ProjW<WT> pw;
  if constexpr (PROJ) {
    // Workgroups b, b + p_rows, ... share a row (and, with 8 rows, an XCD).
    part = bid / a.p_rows;
    bid -= part * a.p_rows;
    pw.load(a, part, threadIdx.x);
  }
  const int hb = bid % a.n_hblocks;
  bid /= a.n_hblocks;
  const int split = bid % a.n_splits;
  const int ridx = bid / a.n_splits;
  const int row = a.rows ? a.rows[ridx] : ridx;
  const int kv_len = min(a.row_pos[row] + 1, a.max_kv);
  const int t0 = split * a.split_tokens;
  if (kv_len <= 0 || t0 >= kv_len) return;
  const int t1 = min(kv_len, t0 + a.split_tokens);
  // A row whose kv_len exceeds the host's max_kv_len bound keeps its first
  // n_splits splits (the grid and workspace cover no more).
  const int nsplit_row = min((kv_len + a.split_tokens - 1) / a.split_tokens, a.n_splits);
  const int* bt = a.bt + (int64_t)(a.row_bt ? a.row_bt[row] : row) * a.bt_stride;
  // Projection epilogue inputs of this thread's column, loaded now.
  [[maybe_unused]] const int pcol = part * 64 + (threadIdx.x >> 3);
  [[maybe_unused]] float p_sc = 1.f, p_bi = 0.f, p_res = 0.f;
  if constexpr (PROJ) {
    if ((threadIdx.x & 7) == 0) {
      if (a.pscale) p_sc = a.pscale[pcol];
      if (a.pbias) p_bi = a.pbias[pcol];
      if (a.pres) p_res = a.pres[(int64_t)row * a.pldr + pcol];
    }
  }

  // The last head block may be partial (n_heads not a multiple of HPB): its
  // lanes past the last head read that head's slice (in bounds) and store
  // nothing.
  const int head = hb * HPB + lane / G;
  const bool head_ok = head < a.n_heads;
  const int sub = lane % G;
  const int D = a.n_heads * kHD;
  const int lane_off = min(head, a.n_heads - 1) * kHD + sub * EPL;

  float q[EPL];
  if (a.q_bf16) {
    const uint16_t* qp = (const uint16_t*)a.q + (int64_t)row * a.ldq + lane_off;
#pragma unroll
    for (int e = 0; e < EPL; ++e) q[e] = bf16_to_f32(qp[e]) * a.qscale;
  } else {
    const float* qp = (const float*)a.q + (int64_t)row * a.ldq + lane_off;
#pragma unroll
    for (int e = 0; e < EPL; ++e) q[e] = qp[e] * a.qscale;
  }

  const int64_t tok_stride = D;                  // elements between consecutive slots
  const int64_t page_stride = tok_stride * kPS;  // elements per page
  const KVT* kbase = (const KVT*)a.kpool + lane_off;
  const KVT* vbase = (const KVT*)a.vpool + lane_off;

  float m = -INFINITY, l = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;

  const int p_first = t0 / kPS, p_last = (t1 - 1) / kPS;
  // The page id of a wave's next page is loaded with the current page's K/V,
  // so its round trip overlaps theirs.
  int id_next = p_first + wave <= p_last ? bt[p_first + wave] : 0;
  for (int p = p_first + wave; p <= p_last; p += NW) {
    int phys = id_next;
    if (p + NW <= p_last) id_next = bt[p + NW];
    phys = min(max(phys, 0), a.num_pages - 1);
    const KVT* kp = kbase + (int64_t)phys * page_stride;
    const KVT* vp = vbase + (int64_t)phys * page_stride;
    uint4 kr[kPS], vr[kPS];
#pragma unroll
    for (int t = 0; t < kPS; ++t) kr[t] = load_stream(kp + t * tok_stride);
#pragma unroll
    for (int t = 0; t < kPS; ++t) vr[t] = load_stream(vp + t * tok_stride);
    const int nvalid = min(kPS, t1 - p * kPS);  // >= 1; < kPS only on the sequence's last page
    float s[kPS];
    float mp = -INFINITY;
#pragma unroll
    for (int t = 0; t < kPS; ++t) {
      float kf[EPL];
      KVTraits<KVT>::unpack(kr[t], kf);
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) d += q[e] * kf[e];
      d = group_sum<G>(d);
      s[t] = (t < nvalid) ? d : -INFINITY;
      mp = fmaxf(mp, s[t]);
    }
    const float mn = fmaxf(m, mp);
    const float corr = fast_exp2(m - mn);
    l *= corr;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] *= corr;
#pragma unroll
    for (int t = 0; t < kPS; ++t) {
      const float pt = fast_exp2(s[t] - mn);
      l += pt;
      float vf[EPL];
      KVTraits<KVT>::unpack(vr[t], vf);
      if (t < nvalid) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] += pt * vf[e];
      }
    }
    m = mn;
  }

  // Merge the NW waves' states through LDS.
  __shared__ float sm[NW][64], sl[NW][64], sacc[NW][EPL][64];
  sm[wave][lane] = m;
  sl[wave][lane] = l;
#pragma unroll
  for (int e = 0; e < EPL; ++e) sacc[wave][e][lane] = acc[e];
  __syncthreads();
  if constexpr (PROJ) {
    // The row's attention output (all heads) into LDS, normalised (and
    // rounded as the separate path stores it), then each thread's share of
    // the projection, summed over the column's 8 threads.
    __shared__ __attribute__((aligned(16))) float so[512];
    if (wave == 0) {
      float M = sm[0][lane];
#pragma unroll
      for (int w = 1; w < NW; ++w) M = fmaxf(M, sm[w][lane]);
      float L = 0.f, O[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) O[e] = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float c = fast_exp2(sm[w][lane] - M);
        L += sl[w][lane] * c;
#pragma unroll
        for (int e = 0; e < EPL; ++e) O[e] += sacc[w][e][lane] * c;
      }
      if (head_ok) {
        const float inv = 1.f / L;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float v = O[e] * inv;
          so[lane_off + e] = a.px_bf16 ? bf16_to_f32(f32_to_bf16(v)) : v;
        }
      }
    }
    __syncthreads();
    float d = pw.dot(a, so + (threadIdx.x & 7) * a.pkpt);
    d += __shfl_xor(d, 1);
    d += __shfl_xor(d, 2);
    d += __shfl_xor(d, 4);
    if ((threadIdx.x & 7) == 0) {
      // cbis_gemm's epilogue order: scale, bias, residual.
      if (a.pscale) d *= p_sc;
      if (a.pbias) d += p_bi;
      if (a.pres) d += p_res;
      a.py[(int64_t)row * a.pldy + pcol] = d;
    }
    return;
  }
  if (wave != 0) return;
  float M = sm[0][lane];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, sm[w][lane]);
  float L = 0.f, O[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) O[e] = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float c = fast_exp2(sm[w][lane] - M);  // waves with no pages: m=-inf -> 0
    L += sl[w][lane] * c;
#pragma unroll
    for (int e = 0; e < EPL; ++e) O[e] += sacc[w][e][lane] * c;
  }
  if (!head_ok) return;
  if (nsplit_row == 1) {
    const float inv = 1.f / L;
    if (a.out_bf16) {
      uint16_t* op = (uint16_t*)a.out + (int64_t)row * a.ldo + lane_off;
#pragma unroll
      for (int e = 0; e < EPL; e += 2) *(uint32_t*)(op + e) = pack_bf16x2(O[e] * inv, O[e + 1] * inv);
    } else {
      float* op = (float*)a.out + (int64_t)row * a.ldo + lane_off;
#pragma unroll
      for (int e = 0; e < EPL; e += 4) *(float4*)(op + e) = make_float4(O[e] * inv, O[e + 1] * inv, O[e + 2] * inv, O[e + 3] * inv);
    }
  } else {
    float* w = a.ws + (((int64_t)ridx * a.n_splits + split) * a.n_heads + head) * kWS;
#pragma unroll
    for (int e = 0; e < EPL; e += 4) *(float4*)(w + sub * EPL + e) = make_float4(O[e], O[e + 1], O[e + 2], O[e + 3]);
    if (sub == 0) {
      w[kHD] = M;
      w[kHD + 1] = L;
    }
  }
}

// Combines split partials: one thread per (row, head, dim), gid in
// [0, n_rows * n_heads * head_dim).
__device__ inline void decode_merge(const DecodeArgs& a, int n_rows, int64_t gid) {
  const int d = (int)(gid % kHD);
  const int64_t rh = gid / kHD;
  const int head = (int)(rh % a.n_heads);
  const int ridx = (int)(rh / a.n_heads);
  if (ridx >= n_rows) return;
  const int row = a.rows ? a.rows[ridx] : ridx;
  const int kv_len = min(a.row_pos[row] + 1, a.max_kv);
  if (kv_len <= 0) return;
  const int ns = min((kv_len + a.split_tokens - 1) / a.split_tokens, a.n_splits);
  if (ns <= 1) return;
  const float* w = a.ws + ((int64_t)ridx * a.n_splits * a.n_heads + head) * kWS;
  const int64_t sstride = (int64_t)a.n_heads * kWS;
  // One pass with a running maximum; the loads of later splits do not depend
  // on the running state, so they are issued ahead.  Split 0 always exists
  // and holds a finite maximum.
  float M = w[kHD], L = w[kHD + 1], O = w[d];
#pragma unroll 4
  for (int s = 1; s < ns; ++s) {
    const float ms = w[s * sstride + kHD], ls = w[s * sstride + kHD + 1], os = w[s * sstride + d];
    const float Mn = fmaxf(M, ms);
    const float c0 = fast_exp2(M - Mn), c1 = fast_exp2(ms - Mn);
    L = L * c0 + ls * c1;
    O = O * c0 + os * c1;
    M = Mn;
  }
  const float r = O / L;
  const int64_t o = (int64_t)row * a.ldo + head * kHD + d;
  if (a.out_bf16) ((uint16_t*)a.out)[o] = f32_to_bf16(r);
  else ((float*)a.out)[o] = r;
}

__global__ __launch_bounds__(256) void paged_decode_merge_kernel(const DecodeArgs a, int n_rows) {
  decode_merge(a, n_rows, (int64_t)blockIdx.x * 256 + threadIdx.x);
}

// The reference-signature attention for page sizes other than kPS (fp32
// Q/K/V/out, head_dim kHD, any page_size > 0; kernels/attention.cu:57-98 takes
// page_size at run time).  One wave per (row, head), four per workgroup.  Lane
// l takes key j = c + l of every 64-key chunk c: it looks up page
// table[j / page_size] and slot j % page_size, forms q.k over the head's 32
// dims from 8 16-byte loads, and the wave runs one online-softmax step per
// chunk (chunk maximum and probability sum by wave reductions, so m and l are
// the same in every lane).  Each lane accumulates p_j v_j over its own keys;
// the 32 output dims are summed across the wave at the end.
__global__ __launch_bounds__(256) void paged_attention_any_page_kernel(const float* __restrict__ Q,
                                                                       const float* __restrict__ kp,
                                                                       const float* __restrict__ vp,
                                                                       const int* __restrict__ table,
                                                                       const int* __restrict__ row_pos,
                                                                       float* __restrict__ out, int total_rows,
                                                                       int n_heads, int page_size, int pages_per_seq,
                                                                       float qscale) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= (int64_t)total_rows * n_heads) return;
  const int row = (int)(unit / n_heads), head = (int)(unit % n_heads);
  const int64_t D = (int64_t)n_heads * kHD;
  const int kv_len = (int)min((int64_t)row_pos[row] + 1, (int64_t)pages_per_seq * page_size);
  if (kv_len <= 0) return;
  const float* qp = Q + row * D + head * kHD;
  float q[kHD];
#pragma unroll
  for (int e = 0; e < kHD; e += 4) {
    const float4 v = *(const float4*)(qp + e);
    q[e] = v.x * qscale; q[e + 1] = v.y * qscale; q[e + 2] = v.z * qscale; q[e + 3] = v.w * qscale;
  }
  const int* tab = table + (int64_t)row * pages_per_seq;
  float m = -INFINITY, l = 0.f, acc[kHD];
#pragma unroll
  for (int e = 0; e < kHD; ++e) acc[e] = 0.f;
  for (int c = 0; c < kv_len; c += 64) {
    const int j = c + lane;
    const bool valid = j < kv_len;
    float s = -INFINITY;
    float4 vv[kHD / 4];
    if (valid) {
      const int64_t slot = ((int64_t)tab[j / page_size] * page_size + j % page_size) * D + head * kHD;
      float4 kk[kHD / 4];
#pragma unroll
      for (int i = 0; i < kHD / 4; ++i) kk[i] = *(const float4*)(kp + slot + 4 * i);
#pragma unroll
      for (int i = 0; i < kHD / 4; ++i) vv[i] = *(const float4*)(vp + slot + 4 * i);
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < kHD / 4; ++i)
        d += q[4 * i] * kk[i].x + q[4 * i + 1] * kk[i].y + q[4 * i + 2] * kk[i].z + q[4 * i + 3] * kk[i].w;
      s = d;
    } else {
#pragma unroll
      for (int i = 0; i < kHD / 4; ++i) vv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float mn = fmaxf(m, wave_max(s));  // finite: lane 0's key is valid
    const float corr = fast_exp2(m - mn);
    const float p = valid ? fast_exp2(s - mn) : 0.f;
    l = l * corr + wave_sum(p);
#pragma unroll
    for (int i = 0; i < kHD / 4; ++i) {
      acc[4 * i] = acc[4 * i] * corr + p * vv[i].x;
      acc[4 * i + 1] = acc[4 * i + 1] * corr + p * vv[i].y;
      acc[4 * i + 2] = acc[4 * i + 2] * corr + p * vv[i].z;
      acc[4 * i + 3] = acc[4 * i + 3] * corr + p * vv[i].w;
    }
    m = mn;
  }
  float mine = 0.f;
#pragma unroll
  for (int e = 0; e < kHD; ++e) {
    const float t = wave_sum(acc[e]);
    if (lane == e) mine = t;
  }
  if (lane < kHD) out[row * D + head * kHD + lane] = mine / l;
}

// ---------------------------------------------------------------------------
// Prefill on MFMA.
// ---------------------------------------------------------------------------
struct PrefillArgs {
  const int* tiles;  // [n_tiles][tile_ints]: first_row, n_valid, bt_row, first_pos (+ 8 page ids)
  int tile_ints;     // 4, or 12 with the tile's first 8 page ids
  const void* q;
  int64_t ldq;
  int q_bf16;
  const uint16_t* kpool;
  const uint16_t* vpool;
  int num_pages;
  const int* bt;
  int64_t bt_stride;
  void* out;
  int64_t ldo;
  int out_bf16;
  int n_heads;
  int max_kv;
  float qscale;  // log2(e) / sqrt(head_dim), folded into Q before its bf16 rounding
};

// Workgroup: one tile of up to 64 query rows x HPW adjacent heads,
// kPrefillWaves waves per head.  A head's waves take its 32-key blocks
// round-robin (block b goes to wave b % kPrefillWaves) and merge their
// softmax states through LDS at the end.  Each wave runs the tile's rows as
// kQG groups of 32 query columns against every key block it loads, so a K/V
// block read from the pages serves 64 queries.  A key's head_dim slice is
// 64 bytes, so adjacent heads of one workgroup read the same 128-byte lines
// at about the same time.  Measured on config 4's two 512-row chunks (one
// layer, isolated): 16.3 us.  Slower: four waves per head (23.1 with one head
// per workgroup, 24.9 with two), a tile pair per workgroup whose waves take
// equal contiguous shares of both tiles' blocks (20.1), four waves per head
// on the long tiles only (20.8 - 24.6: the workgroups' pairing on the CUs is
// lost), deeper K/V rings (17.4 with 3 blocks, 18.8 with 4).
constexpr int kPrefillWaves = 2;  // waves per head
constexpr int kQG = 2;            // 32-query groups per tile
static_assert(32 * kQG == CBIS_PREFILL_TILE_ROWS, "prefill tile rows");
// K/V blocks per wave's register ring: one block in flight while one is
// computed.
constexpr int kPrefillRing = 2;
// Exponent headroom of the lazy softmax rescale (log2 units): p <= 2^8.
constexpr float kLazyRescale = 8.f;

// The two 32-lane halves of v exchanged: each lane gets f(v, v of lane ^ 32)
// through v_permlane32_swap (no LDS round trip).
__device__ inline float2 halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// Workgroups from prefill_blocks on run the decode rows' split merge
// (decode_merge over merge_rows rows) instead: the merge then shares the
// prefill launch, which is independent of it, in place of a launch of its own.
template <int HPW>
__global__ __launch_bounds__(HPW * kPrefillWaves * 64, 2) void paged_prefill_kernel(const PrefillArgs a,
                                                                               const DecodeArgs merge, int merge_rows,
                                                                               unsigned prefill_blocks) {
  if (blockIdx.x >= prefill_blocks) {
    decode_merge(merge, merge_rows, (int64_t)(blockIdx.x - prefill_blocks) * blockDim.x + threadIdx.x);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: block tests and page ids per wave
  const int wave = wave_id % kPrefillWaves;  // key-block lane of this head
  const int hsub = wave_id / kPrefillWaves;
  const int n_hg = a.n_heads / HPW;
  const int tile = blockIdx.x / n_hg;
  const int head = (blockIdx.x % n_hg) * HPW + hsub;
  // The tile descriptor is the same for the whole workgroup: read it into
  // scalar registers, so the tests on it (the causal-mask test per block)
  // compile to scalar branches rather than exec masking.
  // The tile descriptor is the same for the whole workgroup and the page ids
  // of a 32-key block the same for the whole wave: both are read through the
  // constant address space, i.e. with scalar loads (shorter round trips than
  // per-lane loads of one address, and no share of the K/V loads' counter),
  // and the tests on them compile to scalar branches.
  typedef const __attribute__((address_space(4))) int cint_t;
  cint_t* td = (cint_t*)(a.tiles + (int64_t)a.tile_ints * tile);
  const int row0 = td[0], nvalid = td[1], pos0 = td[3];
  cint_t* bt = (cint_t*)(a.bt + (int64_t)td[2] * a.bt_stride);
  const int D = a.n_heads * kHD;
  const int col = lane & 31;  // query index within a group (B / C column)
  const int half = lane >> 5;

  // Q^T of group g as the B operand: lane holds q[32 g + col][half*8 + 0..7]
  // (MFMA 0) and q[32 g + col][16 + half*8 + 0..7] (MFMA 1), bf16.  Rows past
  // the tile's end repeat its last row (computed, never stored).
  bf16x8_t qb0[kQG], qb1[kQG];
  int qpos[kQG];
#pragma unroll
  for (int g = 0; g < kQG; ++g) {
    const int qi = min(32 * g + col, nvalid - 1);
    const int qr = row0 + qi;
    qpos[g] = pos0 + qi;
    float f[16];
    if (a.q_bf16) {
      const uint16_t* qp = (const uint16_t*)a.q + (int64_t)qr * a.ldq + head * kHD;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        f[e] = bf16_to_f32(qp[half * 8 + e]);
        f[8 + e] = bf16_to_f32(qp[16 + half * 8 + e]);
      }
    } else {
      const float* qp = (const float*)a.q + (int64_t)qr * a.ldq + head * kHD;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        f[e] = qp[half * 8 + e];
        f[8 + e] = qp[16 + half * 8 + e];
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qb0[g][e] = (short)f32_to_bf16(f[e] * a.qscale);
      qb1[g][e] = (short)f32_to_bf16(f[8 + e] * a.qscale);
    }
  }
  const int kv_end = min(pos0 + nvalid, a.max_kv);  // keys [0, kv_end) needed by the tile

  // Per-wave V tile [key][dim]: 64-byte rows of four 16-byte chunks, chunk c
  // of key row r in position c ^ ((r >> 2) & 3).  Unswizzled, the 16 lanes
  // of a ds_write_b128 (keys 0..15, one chunk) hit 4 bank groups 4 times
  // each; swizzled, 16 distinct groups.
  __shared__ __attribute__((aligned(16))) uint8_t vt_all[HPW * kPrefillWaves][32 * kHD * 2];
  uint8_t* const vt_w = vt_all[wave_id];
  auto vpos = [](int key, int chunk) { return key * (kHD * 2) + ((chunk ^ ((key >> 2) & 3)) << 4); };
  // Per query column: o (the P.V accumulator), lacc (every entry the
  // column's sum of the bf16-rounded p: an MFMA of an all-ones A with P^T,
  // beside the P.V MFMAs, in place of 16 adds and a lane exchange per block)
  // and the softmax reference m (-inf until the column meets an unmasked
  // key).  negm (every entry -m, or 0 while m = -inf) is the C operand of
  // the score MFMA, so the scores come out relative to m and p = 2^s needs
  // no subtraction per score.
  f32x16_t o[kQG], lacc[kQG], negm[kQG];
  float m[kQG];
  bf16x8_t ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (short)0x3F80;
#pragma unroll
  for (int g = 0; g < kQG; ++g) {
#pragma unroll
    for (int i = 0; i < 16; ++i) o[g][i] = lacc[g][i] = negm[g][i] = 0.f;
    m[g] = -INFINITY;
  }

  // K rows for keys j0 + col in the A-operand layout (lane = key, dims
  // half*8.. and 16 + half*8..) and this lane's half of the key's V row.
  struct KV {
    bf16x8_t k0, k1;
    uint4 v0, v1;
  };
  // A block's 32 keys span two pages.  Each lane reads the page id of its
  // own key (id_of) one block before that block's K/V loads (load_block):
  // the id load then has a whole block of compute to land in, and waiting
  // for it never waits for the K/V loads in flight.
  // Page id of this lane's key j0 + col, clamped to kv_end - 1: keys j0 ..
  // j0 + 15 lie on page min(j0, kv_end - 1) / 16, keys j0 + 16 .. j0 + 31 on
  // page min(j0 + 16, kv_end - 1) / 16 (j0 is a multiple of 32).
  // The ids are clamped to the pool here, in scalar registers.
  auto id_of = [&](int j0) {
    const unsigned last = (unsigned)(kv_end - 1);
    const int pa = min(max(bt[min((unsigned)j0, last) / kPS], 0), a.num_pages - 1);
    const int pb = min(max(bt[min((unsigned)j0 + 16u, last) / kPS], 0), a.num_pages - 1);
    return col < 16 ? pa : pb;
  };
  // Element offset of this lane's key within its page, plus its head:
  // (col % 16) * D + head * kHD for every block that ends before kv_end.
  const int lane_off = (col & (kPS - 1)) * D + head * kHD;
  const int64_t page_elems = (int64_t)kPS * D;
  auto load_block = [&](int j0, int phys, KV& r) {
    int off = lane_off;
    if (j0 + 31 >= kv_end) off = (min(j0 + col, kv_end - 1) & (kPS - 1)) * D + head * kHD;
    const int64_t slot = phys * page_elems + off;
    r.k0 = *(const bf16x8_t*)(a.kpool + slot + half * 8);
    r.k1 = *(const bf16x8_t*)(a.kpool + slot + 16 + half * 8);
    const uint4* vs = (const uint4*)(a.vpool + slot + half * 16);
    r.v0 = vs[0];
    r.v1 = vs[1];
  };
  // ds_read_b64_tr_b16 reads in 16-lane groups: lane i of a group receives
  // element i % 4 of the 8-byte rows addressed by lanes i / 4 + 4 e of the
  // group, e = 0..3.  Lane (group gq, j) addresses key kr = 4 (gq / 2) + j / 4
  // (+ 8, 16, 24), dims 16 (gq % 2) + 4 (j % 4) .. + 3, so lane (dim d, half h)
  // receives V[4 h + e][d] (+ 8, 16, 24): the A-operand layout of V^T below.
  const int kr = 4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2);
  const int dc = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  // Byte offsets of the 8-byte rows read for keys kr + 8 m (m = 0..3) and of
  // this lane's two V chunks (key col, dims 16 half .. + 15).
  int vrd[4];
#pragma unroll
  for (int mm = 0; mm < 4; ++mm) vrd[mm] = vpos(kr + 8 * mm, dc >> 3) + (dc & 7) * 2;
  const int vwr0 = vpos(col, 2 * half), vwr1 = vpos(col, 2 * half + 1);
  auto vt_read = [&](int mm) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4_t*)(__attribute__((address_space(3))) void*)(vt_w + vrd[mm]));
  };
  auto compute_block = [&](int j0, const KV& r) {
    *(uint4*)(vt_w + vwr0) = r.v0;  // this lane's key, dims 16 half .. + 7
    *(uint4*)(vt_w + vwr1) = r.v1;  // and + 8 .. + 15
    bf16x8_t pb0[kQG], pb1[kQG];
    // Both groups' scores first (no branch between their MFMAs), then one
    // uniform mask test and one uniform rescale test for the block.
    // s[g][i]: key j0 + 8*(i/4) + 4*half + (i%4), query 32 g + col, in log2
    // units relative to m: q.k * log2(e)/sqrt(hd) - m (the scale is folded
    // into Q).  Only blocks reaching past the tile's first query position or
    // past kv_end need the causal mask.
    f32x16_t s[kQG];
#pragma unroll
    for (int g = 0; g < kQG; ++g) {
      s[g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(r.k0, qb0[g], negm[g], 0, 0, 0);
      s[g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(r.k1, qb1[g], s[g], 0, 0, 0);
    }
    if (j0 + 31 > pos0 || j0 + 31 >= kv_end) {
#pragma unroll
      for (int g = 0; g < kQG; ++g)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kj = j0 + 8 * (i >> 2) + 4 * half + (i & 3);
          if (kj > qpos[g] || kj >= kv_end) s[g][i] = -INFINITY;
        }
    }
    float smax[kQG], thr[kQG];
    bool up[kQG];
#pragma unroll
    for (int g = 0; g < kQG; ++g) {
      float v = s[g][0];
#pragma unroll
      for (int i = 1; i < 16; ++i) v = fmaxf(v, s[g][i]);
      const float2 h = halves(v);
      smax[g] = fmaxf(h.x, h.y);
      thr[g] = m[g] == -INFINITY ? -INFINITY : kLazyRescale;
      up[g] = smax[g] > thr[g];
    }
    // Lazy rescaling: m is raised -- o and lacc rescaled by 2^(m_old - m_new),
    // the block's scores shifted, negm reloaded -- only when some column's
    // block maximum exceeds it by more than kLazyRescale (log2 units), or on
    // a column's first unmasked key.  Otherwise p = 2^s <= 2^8, well inside
    // fp32 and bf16.  In exact arithmetic the result does not depend on the
    // reference; the wave merge below combines each wave's (m, l, o) by its
    // own reference.  A column whose keys are all masked so far keeps
    // m = -inf and p = 0.
    if (__builtin_amdgcn_ballot_w64(up[0] || up[1]) != 0) {
#pragma unroll
      for (int g = 0; g < kQG; ++g) {
        const float cur = m[g] == -INFINITY ? 0.f : m[g];
        const float mn = up[g] ? fmaxf(m[g], smax[g] + cur) : m[g];
        const float corr = (up[g] && m[g] != -INFINITY) ? fast_exp2(m[g] - mn) : 1.f;
        const float d = up[g] ? mn - cur : 0.f;
        const float nm = mn == -INFINITY ? 0.f : -mn;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          s[g][i] -= d;
          o[g][i] *= corr;
          lacc[g][i] *= corr;
          negm[g][i] = nm;
        }
        m[g] = mn;
      }
    }
#pragma unroll
    for (int g = 0; g < kQG; ++g) {
      float pf[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) pf[i] = fast_exp2(s[g][i]);
      uint4 u0, u1;
      u0.x = pack_bf16x2(pf[0], pf[1]);   u0.y = pack_bf16x2(pf[2], pf[3]);
      u0.z = pack_bf16x2(pf[4], pf[5]);   u0.w = pack_bf16x2(pf[6], pf[7]);
      u1.x = pack_bf16x2(pf[8], pf[9]);   u1.y = pack_bf16x2(pf[10], pf[11]);
      u1.z = pack_bf16x2(pf[12], pf[13]); u1.w = pack_bf16x2(pf[14], pf[15]);
      pb0[g] = __builtin_bit_cast(bf16x8_t, u0);
      pb1[g] = __builtin_bit_cast(bf16x8_t, u1);
    }
    // V^T as the A operand: lane = dim (col), k-slot e of MFMA b holds key
    // 16*b + 8*(e/4) + 4*half + (e%4), matching P's register order.  The V
    // tile is this wave's own: its LDS writes are complete (lgkmcnt) before
    // its lanes read each other's entries.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    const short4_t a0 = vt_read(0), a1 = vt_read(1), b0 = vt_read(2), b1 = vt_read(3);
    bf16x8_t va0, va1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      va0[e] = a0[e]; va0[4 + e] = a1[e];
      va1[e] = b0[e]; va1[4 + e] = b1[e];
    }
#pragma unroll
    for (int g = 0; g < kQG; ++g) {
      o[g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va0, pb0[g], o[g], 0, 0, 0);
      o[g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va1, pb1[g], o[g], 0, 0, 0);
      lacc[g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ones, pb0[g], lacc[g], 0, 0, 0);
      lacc[g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ones, pb1[g], lacc[g], 0, 0, 0);
    }
    // The next block's V writes come after these reads in program order.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  };

  // This wave's key blocks (wave, wave + kPrefillWaves, ...) stream through
  // a kPrefillRing-entry register ring: its block i + kPrefillRing - 1 is in
  // flight while block i is computed, and the page ids of block
  // i + kPrefillRing with it (ids[i % kPrefillRing]).  Loads past the last
  // block are clamped to key kv_end - 1 (in bounds) and left unused.
  const int nblk = (kv_end + 31) / 32;
  const int nmine = nblk > wave ? (nblk - wave + kPrefillWaves - 1) / kPrefillWaves : 0;
  auto key0 = [&](int i) { return 32 * (wave + kPrefillWaves * i); };
  constexpr int R = kPrefillRing;
  KV ring[R];
  int ids[R];
  if (a.tile_ints == 12) {
    // The first R blocks' page ids come with the tile descriptor (entries
    // 4 + j0 / 16 and the next: pages min(j0, kv_end - 1) / 16 and
    // min(j0 + 16, kv_end - 1) / 16, as id_of reads them), so their K/V
    // loads follow the descriptor's round trip directly.
    static_assert(32 * (kPrefillWaves * (kPrefillRing - 1) + kPrefillWaves - 1) / 16 + 1 < 8, "descriptor pages");
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int k = key0(u) / 16;
      const int pa = min(max(td[4 + k], 0), a.num_pages - 1);
      const int pb = min(max(td[5 + k], 0), a.num_pages - 1);
      ids[u] = col < 16 ? pa : pb;
    }
  } else {
#pragma unroll
    for (int u = 0; u < R; ++u) ids[u] = id_of(key0(u));
  }
#pragma unroll
  for (int u = 0; u < R - 1; ++u) load_block(key0(u), ids[u], ring[u]);
  for (int i0 = 0; i0 < nmine; i0 += R) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
      ids[u] = id_of(key0(i0 + u + R));
      load_block(key0(i0 + u + R - 1), ids[(u + R - 1) % R], ring[(u + R - 1) % R]);
      if (i0 + u < nmine) compute_block(key0(i0 + u), ring[u]);
    }
  }

  // Merge the waves' (m, l, o) per query column; a wave without blocks has
  // m = -inf and contributes nothing.  Wave 0 always holds key 0.
  __shared__ float pm_all[HPW][kPrefillWaves][kQG][64], pl_all[HPW][kPrefillWaves][kQG][64];
  __shared__ f32x16_t po_all[HPW][kPrefillWaves - 1][kQG][64];
#pragma unroll
  for (int g = 0; g < kQG; ++g) {
    pm_all[hsub][wave][g][lane] = m[g];
    pl_all[hsub][wave][g][lane] = lacc[g][0];
    if (wave > 0) po_all[hsub][wave - 1][g][lane] = o[g];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int g = 0; g < kQG; ++g) {
    float l = lacc[g][0];
    float M = m[g];
#pragma unroll
    for (int w = 1; w < kPrefillWaves; ++w) M = fmaxf(M, pm_all[hsub][w][g][lane]);
    {
      const float c0 = fast_exp2(m[g] - M);
      l *= c0;
#pragma unroll
      for (int i = 0; i < 16; ++i) o[g][i] *= c0;
    }
#pragma unroll
    for (int w = 1; w < kPrefillWaves; ++w) {
      const float c = fast_exp2(pm_all[hsub][w][g][lane] - M);
      l += pl_all[hsub][w][g][lane] * c;
      const f32x16_t ow = po_all[hsub][w - 1][g][lane];
#pragma unroll
      for (int i = 0; i < 16; ++i) o[g][i] += ow[i] * c;
    }
    // o[g][i]: dim 8*(i/4) + 4*half + (i%4) of query 32 g + col.
    // Dims 8 b + 4 half .. + 3 are o[g][4 b .. 4 b + 3]: one 8-byte (bf16) or
    // 16-byte (fp32) store each (ldo % 4 == 0 and a 16-byte aligned out).
    const int qi = 32 * g + col;
    if (qi < nvalid) {
      const float inv = 1.f / l;
      const int64_t ob = (int64_t)(row0 + qi) * a.ldo + head * kHD + 4 * half;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float v0 = o[g][4 * b] * inv, v1 = o[g][4 * b + 1] * inv, v2 = o[g][4 * b + 2] * inv,
                    v3 = o[g][4 * b + 3] * inv;
        if (a.out_bf16)
          *(uint2*)((uint16_t*)a.out + ob + 8 * b) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
        else
          *(float4*)((float*)a.out + ob + 8 * b) = make_float4(v0, v1, v2, v3);
      }
    }
  }
}

int resolve_split(const cbis_attn_desc* d, int hblocks, int* n_splits) {
  int split = d->split_tokens;
  const int max_kv = std::max(1, d->max_kv_len);
  if (split <= 0) {
    if (d->max_kv_len <= 0) {
      split = 1 << 30;  // single pass
    } else {
      const int64_t units = (int64_t)std::max(1, d->n_rows) * hblocks;
      const int64_t pages = units * cdiv(max_kv, kPS);  // upper bound of the call's page loads
      if (pages <= 8 * kResidentWaves) {
        // Small call (a few pages per resident wave): one round of fat
        // workgroups, 6 pages per wave; per-workgroup setup, partial writes
        // and the merge weigh more than the tail here.
        split = (int)std::min<int64_t>(max_kv, 8 * 6 * kPS);
      } else {
        // Aim for >= 2048 workgroups across the chip.
        const int64_t want = std::max<int64_t>(1, cdiv(2048, units));
        int64_t s = cdiv(max_kv, want);
        s = std::max<int64_t>(64, cdiv(s, 64) * 64);
        split = (int)std::min<int64_t>(s, 1 << 30);
      }
    }
  }
  *n_splits = (int)cdiv(max_kv, split);
  if (*n_splits < 1) *n_splits = 1;
  return split;
}

// Head blocks of a decode call: 1 KiB of one token's K (or V) row each, 8
// heads of fp32 or 16 of bf16; the last one may be partial.
int head_blocks(const cbis_attn_desc* d) {
  const int hpb = d->kv_dtype == CBIS_F32 ? 8 : 16;
  return (int)cdiv(d->n_heads, hpb);
}

int validate(const cbis_attn_desc* d, const char* who, bool need_out = true) {
  CBIS_REQUIRE(d, CBIS_ERR_INVALID, "%s: null descriptor", who);
  CBIS_REQUIRE(d->head_dim == kHD && d->page_size == kPS, CBIS_ERR_UNSUPPORTED,
               "%s: head_dim %d / page_size %d (this build supports 32 / 16)", who, d->head_dim, d->page_size);
  CBIS_REQUIRE(d->kv_dtype == CBIS_F32 || d->kv_dtype == CBIS_BF16, CBIS_ERR_UNSUPPORTED, "%s: kv dtype", who);
  CBIS_REQUIRE(d->n_heads > 0, CBIS_ERR_INVALID, "%s: n_heads %d", who, d->n_heads);
  CBIS_REQUIRE(d->split_tokens <= 0 || d->split_tokens % kPS == 0, CBIS_ERR_INVALID,
               "%s: split_tokens %d must be a multiple of page_size %d", who, d->split_tokens, kPS);
  CBIS_REQUIRE(d->q_dtype == CBIS_F32 || d->q_dtype == CBIS_BF16, CBIS_ERR_UNSUPPORTED, "%s: q dtype", who);
  CBIS_REQUIRE(d->out_dtype == CBIS_F32 || d->out_dtype == CBIS_BF16, CBIS_ERR_UNSUPPORTED, "%s: out dtype", who);
  CBIS_REQUIRE(d->n_rows >= 0 && d->num_pages > 0 && d->bt_stride > 0, CBIS_ERR_INVALID, "%s: bad sizes", who);
  CBIS_REQUIRE(d->q && d->k_pool && d->v_pool && d->block_table && (d->out || !need_out), CBIS_ERR_INVALID,
               "%s: null pointer", who);
  if (need_out)
    CBIS_REQUIRE(d->ldo % 4 == 0 && ((uintptr_t)d->out & 15u) == 0, CBIS_ERR_INVALID,
                 "%s: out rows must be 16-byte aligned", who);
  CBIS_REQUIRE(((uintptr_t)d->k_pool & 15u) == 0 && ((uintptr_t)d->v_pool & 15u) == 0, CBIS_ERR_INVALID,
               "%s: pools must be 16-byte aligned", who);
  return CBIS_OK;
}

// Launches the decode kernel for d's rows (d validated, n_rows > 0) with the
// split partials in ws (ws_bytes long; d->workspace is not read); *m gets
// its arguments and *ns its split count -- the split merge is the caller's.
int decode_launch(const cbis_attn_desc* d, void* ws, size_t ws_bytes, hipStream_t s, DecodeArgs* m, int* ns_out,
                  const char* who) {
  const int hblocks = head_blocks(d);
  int ns = 1;
  const int split = resolve_split(d, hblocks, &ns);
  if (ns > 1) {
    const size_t need = (size_t)d->n_rows * ns * d->n_heads * kWS * sizeof(float);
    CBIS_REQUIRE(ws && ws_bytes >= need, CBIS_ERR_WORKSPACE, "%s: workspace %zu bytes, need %zu", who, ws_bytes,
                 need);
  }
  DecodeArgs a;
  a.rows = d->rows;
  a.q = d->q;
  a.ldq = d->ldq;
  a.q_bf16 = d->q_dtype == CBIS_BF16;
  a.kpool = d->k_pool;
  a.vpool = d->v_pool;
  a.num_pages = d->num_pages;
  a.bt = d->block_table;
  a.bt_stride = d->bt_stride;
  a.row_bt = d->row_bt;
  a.row_pos = d->row_pos;
  a.out = d->out;
  a.ldo = d->ldo;
  a.out_bf16 = d->out_dtype == CBIS_BF16;
  a.ws = (float*)ws;
  a.n_heads = d->n_heads;
  a.n_hblocks = hblocks;
  a.n_splits = ns;
  a.split_tokens = split;
  a.max_kv = (int)std::min<int64_t>(d->bt_stride * kPS, 1 << 30);
  a.qscale = kLog2e / sqrtf((float)kHD);
  const int64_t grid = (int64_t)d->n_rows * ns * hblocks;
  CBIS_REQUIRE(grid < (1LL << 31), CBIS_ERR_UNSUPPORTED, "%s: grid too large", who);
  // 16 waves per workgroup, each wave half the pages of an 8-wave one, for
  // one pass per row over at least one workgroup per CU (config 4, 768
  // workgroups: 523 us against 536) and for split calls of at least two
  // workgroups per CU (config 3, 768 workgroups: 5.83 TB/s against
  // 5.68-5.75).  Split calls of one workgroup per CU keep 8 waves (config 5,
  // 256 workgroups: 10.83 ms per step with 16 against 10.80).
  const bool wide = grid >= 256 && (ns == 1 || grid >= 512);
  if (d->kv_dtype == CBIS_F32) {
    if (wide) paged_decode_kernel<float, 16><<<(unsigned)grid, 1024, 0, s>>>(a);
    else paged_decode_kernel<float, 8><<<(unsigned)grid, 512, 0, s>>>(a);
  } else {
    if (wide) paged_decode_kernel<uint16_t, 16><<<(unsigned)grid, 1024, 0, s>>>(a);
    else paged_decode_kernel<uint16_t, 8><<<(unsigned)grid, 512, 0, s>>>(a);
  }
  *m = a;
  *ns_out = ns;
  return check_launch(who);
}

int merge_launch(const DecodeArgs& m, int n_rows, hipStream_t s) {
  const int64_t threads = (int64_t)n_rows * m.n_heads * kHD;
  paged_decode_merge_kernel<<<(unsigned)cdiv(threads, 256), 256, 0, s>>>(m, n_rows);
  return check_launch("cbis_paged_attention(merge)");
}

// Split-KV decode over d's rows with the partials in ws: the decode launch,
// then the merge launch when a row takes more than one split.
int paged_attention_ws(const cbis_attn_desc* d, void* ws, size_t ws_bytes, hipStream_t s, const char* who) {
  int rc = validate(d, who);
  if (rc) return rc;
  CBIS_REQUIRE(d->row_pos, CBIS_ERR_INVALID, "%s: null row_pos", who);
  if (d->n_rows == 0) return CBIS_OK;
  DecodeArgs m;
  int ns = 1;
  rc = decode_launch(d, ws, ws_bytes, s, &m, &ns, who);
  if (rc || ns <= 1) return rc;
  return merge_launch(m, d->n_rows, s);
}

// Decode attention + out-projection in one launch (cbis_paged_attention_proj).
int attention_proj(const cbis_attn_desc* d, const cbis_gemm_desc* g, hipStream_t s) {
  const char* who = "cbis_paged_attention_proj";
  int rc = validate(d, who, false);
  if (rc) return rc;
  CBIS_REQUIRE(d->row_pos && g, CBIS_ERR_INVALID, "%s: null row_pos / projection", who);
  const int D = d->n_heads * kHD;
  const int wbytes = g->w_dtype == CBIS_F32 ? 4 : g->w_dtype == CBIS_BF16 ? 2 : 0;
  CBIS_REQUIRE(head_blocks(d) == 1 && D % 64 == 0 && wbytes && D * wbytes <= 1024, CBIS_ERR_UNSUPPORTED,
               "%s: %d heads of %s K/V with %s weights (needs one head block, n_heads * head_dim a multiple of "
               "64, at most 256 with fp32 weights or 512 with bf16)",
               who, d->n_heads, d->kv_dtype == CBIS_F32 ? "fp32" : "bf16",
               g->w_dtype == CBIS_F32 ? "fp32" : g->w_dtype == CBIS_BF16 ? "bf16" : "other");
  CBIS_REQUIRE(g->N == D && g->K == D, CBIS_ERR_INVALID, "%s: projection N %d, K %d must equal n_heads * head_dim %d",
               who, g->N, g->K, D);
  CBIS_REQUIRE(g->y_dtype == CBIS_F32 && (g->x_dtype == CBIS_F32 || g->x_dtype == CBIS_BF16) &&
                   g->epilogue == CBIS_EPI_NONE && !g->k_pool && !g->v_pool,
               CBIS_ERR_UNSUPPORTED, "%s: fp32 Y, fp32 / bf16 X, no GELU, no K/V scatter", who);
  CBIS_REQUIRE(g->W && g->Y && (!g->residual || g->ldr >= D) && g->ldy >= D, CBIS_ERR_INVALID,
               "%s: null W / Y or short rows", who);
  CBIS_REQUIRE(((uintptr_t)g->W & 15u) == 0 && g->ldw >= D && (g->ldw * wbytes) % 16 == 0, CBIS_ERR_INVALID,
               "%s: W must be 16-byte aligned with 16-byte row pitch", who);
  if (d->n_rows == 0) return CBIS_OK;
  DecodeArgs a = {};
  a.rows = d->rows;
  a.q = d->q;
  a.ldq = d->ldq;
  a.q_bf16 = d->q_dtype == CBIS_BF16;
  a.kpool = d->k_pool;
  a.vpool = d->v_pool;
  a.num_pages = d->num_pages;
  a.bt = d->block_table;
  a.bt_stride = d->bt_stride;
  a.row_bt = d->row_bt;
  a.row_pos = d->row_pos;
  a.n_heads = d->n_heads;
  a.n_hblocks = 1;
  a.n_splits = 1;
  a.split_tokens = 1 << 30;  // one pass per row
  a.max_kv = (int)std::min<int64_t>(d->bt_stride * kPS, 1 << 30);
  a.qscale = kLog2e / sqrtf((float)kHD);
  a.pw = g->W;
  a.pldw = g->ldw;
  a.pscale = g->w_scale;
  a.pbias = g->bias;
  a.pres = g->residual;
  a.pldr = g->ldr;
  a.py = (float*)g->Y;
  a.pldy = g->ldy;
  a.p_rows = d->n_rows;
  a.pkpt = D / 8;
  a.px_bf16 = g->x_dtype == CBIS_BF16;
  const int64_t grid = (int64_t)d->n_rows * (D / 64);
  CBIS_REQUIRE(grid < (1LL << 31), CBIS_ERR_UNSUPPORTED, "%s: grid too large", who);
  if (d->kv_dtype == CBIS_F32) {
    if (g->w_dtype == CBIS_F32) paged_decode_kernel<float, 8, float><<<(unsigned)grid, 512, 0, s>>>(a);
    else paged_decode_kernel<float, 8, uint16_t><<<(unsigned)grid, 512, 0, s>>>(a);
  } else {
    if (g->w_dtype == CBIS_F32) paged_decode_kernel<uint16_t, 8, float><<<(unsigned)grid, 512, 0, s>>>(a);
    else paged_decode_kernel<uint16_t, 8, uint16_t><<<(unsigned)grid, 512, 0, s>>>(a);
  }
  return check_launch(who);
}

// Split-KV partials of cbis_paged_attention_static: a file-scope device
// array, so that entry point allocates nothing.  Each GPU the library runs
// on holds its own copy (32 MiB) until the process ends.  In host code the
// array's name is not a device address: its address on the current device
// is looked up once per device with hipGetSymbolAddress and kept in
// g_scratch_dev, and only that address reaches the kernels.  The decode
// kernel writes every partial the merge reads in the same call, so nothing
// in it needs to start at zero.
constexpr size_t kStaticScratchBytes = CBIS_ATTN_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kStaticScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

int static_scratch(void** out, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  CBIS_REQUIRE(e == hipSuccess, CBIS_ERR_HIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  CBIS_REQUIRE(dev >= 0 && dev < kMaxDevices, CBIS_ERR_UNSUPPORTED, "%s: device %d", who, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    CBIS_REQUIRE(e == hipSuccess && p, CBIS_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                 hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return CBIS_OK;
}

int check_tiles(const cbis_attn_desc* d, int n_tiles, const int* tiles, const char* who) {
  CBIS_REQUIRE(n_tiles >= 0, CBIS_ERR_INVALID, "%s: n_tiles < 0", who);
  if (n_tiles == 0) return CBIS_OK;
  CBIS_REQUIRE(d->kv_dtype == CBIS_BF16, CBIS_ERR_UNSUPPORTED, "%s: prefill tiles need bf16 K/V", who);
  CBIS_REQUIRE(tiles && ((uintptr_t)tiles & 15u) == 0, CBIS_ERR_INVALID,
               "%s: tiles must be a 16-byte aligned device array", who);
  CBIS_REQUIRE(d->tile_pages == 0 || d->tile_pages == 8, CBIS_ERR_INVALID, "%s: tile_pages %d (0 or 8)", who,
               d->tile_pages);
  return CBIS_OK;
}

// Launches the prefill kernel for n_tiles > 0 tiles; with merge_rows > 0 the
// launch also runs the split merge of the decode kernel launched before it
// (arguments *m).
int prefill_launch(const cbis_attn_desc* d, int n_tiles, const int* tiles, hipStream_t s, const DecodeArgs* m,
                   int merge_rows, const char* who) {
  PrefillArgs a;
  a.tiles = tiles;
  a.tile_ints = d->tile_pages == 8 ? 12 : 4;
  a.q = d->q;
  a.ldq = d->ldq;
  a.q_bf16 = d->q_dtype == CBIS_BF16;
  a.kpool = (const uint16_t*)d->k_pool;
  a.vpool = (const uint16_t*)d->v_pool;
  a.num_pages = d->num_pages;
  a.bt = d->block_table;
  a.bt_stride = d->bt_stride;
  a.out = d->out;
  a.ldo = d->ldo;
  a.out_bf16 = d->out_dtype == CBIS_BF16;
  a.n_heads = d->n_heads;
  a.max_kv = (int)std::min<int64_t>(d->bt_stride * kPS, 1 << 30);
  a.qscale = kLog2e / sqrtf((float)kHD);
  // Two heads per workgroup (four waves).
  const int hpw = d->n_heads % 2 == 0 ? 2 : 1;
  const int block = hpw * kPrefillWaves * 64;
  const int64_t pgrid = (int64_t)n_tiles * (d->n_heads / hpw);
  const DecodeArgs none = {};
  const int64_t mgrid = merge_rows > 0 ? cdiv((int64_t)merge_rows * m->n_heads * kHD, block) : 0;
  CBIS_REQUIRE(pgrid + mgrid < (1LL << 31), CBIS_ERR_UNSUPPORTED, "%s: grid too large", who);
  const DecodeArgs& mm = merge_rows > 0 ? *m : none;
  if (hpw == 2) paged_prefill_kernel<2><<<(unsigned)(pgrid + mgrid), block, 0, s>>>(a, mm, merge_rows, (unsigned)pgrid);
  else paged_prefill_kernel<1><<<(unsigned)(pgrid + mgrid), block, 0, s>>>(a, mm, merge_rows, (unsigned)pgrid);
  return check_launch(who);
}

}  // namespace
}  // namespace cbis

using namespace cbis;

extern "C" {

size_t cbis_paged_attention_workspace_size(const cbis_attn_desc* d) {
  if (!d || d->head_dim != kHD || d->n_heads <= 0) return 0;
  if (d->split_tokens > 0 && d->split_tokens % kPS != 0) return 0;  // refused by the launch
  int ns = 1;
  resolve_split(d, head_blocks(d), &ns);
  if (ns <= 1) return 0;
  return (size_t)d->n_rows * ns * d->n_heads * kWS * sizeof(float);
}

int cbis_paged_attention(const cbis_attn_desc* d, cbis_stream_t stream) {
  return paged_attention_ws(d, d ? d->workspace : nullptr, d ? d->workspace_bytes : 0, (hipStream_t)stream,
                            "cbis_paged_attention");
}

int cbis_paged_attention_proj(const cbis_attn_desc* d, const cbis_gemm_desc* proj, cbis_stream_t stream) {
  return attention_proj(d, proj, (hipStream_t)stream);
}

int cbis_paged_attention_static(const cbis_attn_desc* d, cbis_stream_t stream) {
  const char* who = "cbis_paged_attention_static";
  int rc = validate(d, who);
  if (rc) return rc;
  void* ws = nullptr;
  if ((rc = static_scratch(&ws, who))) return rc;
  const size_t need = cbis_paged_attention_workspace_size(d);
  CBIS_REQUIRE(need <= kStaticScratchBytes, CBIS_ERR_WORKSPACE,
               "%s: the call's split partials take %zu bytes, more than the %zu-byte static scratch", who, need,
               kStaticScratchBytes);
  return paged_attention_ws(d, ws, kStaticScratchBytes, (hipStream_t)stream, who);
}

int cbis_paged_prefill_attention(const cbis_attn_desc* d, int n_tiles, const int* tiles, cbis_stream_t stream) {
  int rc = validate(d, "cbis_paged_prefill_attention");
  if (rc) return rc;
  rc = check_tiles(d, n_tiles, tiles, "cbis_paged_prefill_attention");
  if (rc || n_tiles == 0) return rc;
  return prefill_launch(d, n_tiles, tiles, (hipStream_t)stream, nullptr, 0, "cbis_paged_prefill_attention");
}

int cbis_paged_attention_mixed(const cbis_attn_desc* d, int n_tiles, const int* tiles, cbis_stream_t stream) {
  const char* who = "cbis_paged_attention_mixed";
  int rc = validate(d, who);
  if (rc) return rc;
  rc = check_tiles(d, n_tiles, tiles, who);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  DecodeArgs m = {};
  int ns = 1;
  if (d->n_rows > 0) {
    CBIS_REQUIRE(d->row_pos, CBIS_ERR_INVALID, "%s: null row_pos", who);
    rc = decode_launch(d, d->workspace, d->workspace_bytes, s, &m, &ns, who);
    if (rc) return rc;
  }
  const int merge_rows = ns > 1 ? d->n_rows : 0;
  if (n_tiles > 0) return prefill_launch(d, n_tiles, tiles, s, &m, merge_rows, who);
  return merge_rows ? merge_launch(m, merge_rows, s) : CBIS_OK;
}

int cbis_fused_paged_causal_attention(const float* Q, const float* kp, const float* vp, const int* row_page_table,
                                      const int* row_query_pos, float* out, int total_rows, int n_heads, int head_dim,
                                      int page_size, int pages_per_seq, cbis_stream_t stream) {
  if (page_size != kPS && head_dim == kHD) {
    const char* who = "cbis_fused_paged_causal_attention";
    CBIS_REQUIRE(total_rows >= 0 && n_heads > 0 && page_size > 0 && pages_per_seq > 0, CBIS_ERR_INVALID,
                 "%s: total_rows %d, n_heads %d, page_size %d, pages_per_seq %d", who, total_rows, n_heads, page_size,
                 pages_per_seq);
    CBIS_REQUIRE(Q && kp && vp && row_page_table && row_query_pos && out, CBIS_ERR_INVALID, "%s: null pointer", who);
    CBIS_REQUIRE(((uintptr_t)Q & 15u) == 0 && ((uintptr_t)kp & 15u) == 0 && ((uintptr_t)vp & 15u) == 0, CBIS_ERR_INVALID,
                 "%s: Q and the pools must be 16-byte aligned", who);
    const int64_t units = (int64_t)total_rows * n_heads;
    if (units == 0) return CBIS_OK;
    CBIS_REQUIRE(cdiv(units, 4) < (1LL << 31), CBIS_ERR_UNSUPPORTED, "%s: grid too large", who);
    paged_attention_any_page_kernel<<<(unsigned)cdiv(units, 4), 256, 0, (hipStream_t)stream>>>(
        Q, kp, vp, row_page_table, row_query_pos, out, total_rows, n_heads, page_size, pages_per_seq,
        kLog2e / sqrtf((float)kHD));
    return check_launch(who);
  }
  cbis_attn_desc d = {};
  d.n_rows = total_rows;
  d.n_heads = n_heads;
  d.head_dim = head_dim;
  d.page_size = page_size;
  d.q_dtype = CBIS_F32;
  d.q = Q;
  d.ldq = (int64_t)n_heads * head_dim;
  d.kv_dtype = CBIS_F32;
  d.k_pool = kp;
  d.v_pool = vp;
  d.num_pages = 0x7FFFFFFF;  // the reference launcher carries no pool size
  d.block_table = row_page_table;
  d.bt_stride = pages_per_seq;
  d.row_pos = row_query_pos;
  d.out_dtype = CBIS_F32;
  d.out = out;
  d.ldo = (int64_t)n_heads * head_dim;
  d.max_kv_len = 0;  // single pass, no workspace
  return cbis_paged_attention(&d, stream);
}

}  // extern "C"
