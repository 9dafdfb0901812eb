// Device and host helpers shared by the gfx950 kernels: vector types, bf16
// and OCP fp8-e4m3 codecs, wave64 cross-lane reductions (DPP), the
// synthetic-data PRNG, and the C-ABI error plumbing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/cbis_kernels.h"

namespace cbis {

typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Error reporting for the C-ABI.
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---------------------------------------------------------------------------
// bf16 / fp8.
// ---------------------------------------------------------------------------
__host__ __device__ inline float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round to nearest even; NaN stays a quiet NaN.  On the device this is
// gfx950's v_cvt_pk_bf16_f32 (round to nearest even); the host restates it.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
#ifdef __HIP_DEVICE_COMPILE__
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
#endif
}

__device__ inline float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__host__ __device__ inline uint32_t pack_bf16x2(float a, float b) {
#ifdef __HIP_DEVICE_COMPILE__
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
#else
  return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
#endif
}

// OCP e4m3 -> bf16 bits, exact for every finite code (e4m3 values are a
// subset of bf16).  Normal codes move the exponent from bias 7 to bias 127
// (+120) and widen the 3-bit mantissa; subnormal codes m * 2^-9 (m = 1..7)
// are normalised by the position of m's leading one.  NaN (S.1111.111) maps
// to a bf16 quiet NaN.
__host__ __device__ inline uint16_t e4m3_to_bf16(uint32_t b) {
  const uint32_t s = (b & 0x80u) << 8;
  const uint32_t e = (b >> 3) & 0xFu;
  const uint32_t m = b & 7u;
  if (e == 0xFu && m == 7u) return (uint16_t)(s | 0x7FC0u);
  if (e != 0u) return (uint16_t)(s | ((e + 120u) << 7) | (m << 4));
  if (m == 0u) return (uint16_t)s;
  // m * 2^-9: leading one at bit p (0..2) -> value 2^(p-9) * (1 + rest/2^p)
  const uint32_t p = (m >= 4u) ? 2u : (m >= 2u ? 1u : 0u);
  const uint32_t rest = m & ((1u << p) - 1u);
  return (uint16_t)(s | ((p - 9u + 127u) << 7) | (rest << (7u - p)));
}

// fp32 -> OCP e4m3, round to nearest even, saturating to +-448 (NaN -> 0x7F).
// Works on the fp32 bit pattern: the value is re-expressed in units of the
// e4m3 quantum of its binade and rounded with the usual (half + lsb) rule.
__host__ __device__ inline uint8_t f32_to_e4m3(float f) {
  uint32_t u = __float_as_uint(f);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  u &= 0x7FFFFFFFu;
  if (u > 0x7F800000u) return 0x7F;
  if (u >= 0x43E00000u) return sign | 0x7E;  // |f| >= 448
  const int exp = (int)(u >> 23) - 127;
  if (exp < -6) {
    // subnormal e4m3 range: quantum 2^-9; q = rne(|f| * 2^9) in [0, 8]
    if (exp < -11) return sign;  // |f| < 2^-11 rounds to 0 (< half quantum)
    const uint32_t mant = (u & 0x7FFFFFu) | 0x800000u;  // |f| = mant * 2^(exp-23)
    const int shift = 23 - (exp + 9);                   // bits below the 2^-9 quantum
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return sign | (uint8_t)q;  // q == 8 is the smallest normal code
  }
  // normal: keep 3 mantissa bits, round on the remaining 20
  uint32_t mant = u & 0x7FFFFFu;
  uint32_t e = (uint32_t)(exp + 7);
  uint32_t q = mant >> 20;
  const uint32_t rem = mant & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ++q;
  if (q == 8u) { q = 0u; ++e; }
  uint32_t code = (e << 3) | q;
  if (code > 0x7Eu) code = 0x7Eu;
  return sign | (uint8_t)code;
}

// ---------------------------------------------------------------------------
// PRNG spec: counter-based splitmix64; exact Irwin-Hall(12) normals.
// ---------------------------------------------------------------------------
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ULL;

__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t prng_key(uint64_t seed, uint64_t stream) {
  return mix64(seed + kGolden * (mix64(stream + kGolden) | 1ULL));
}

__host__ __device__ inline uint64_t prng_u64(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGolden); }

// Sum of 12 centred 24-bit uniforms minus 6, as the exact double
// (2*S + 12 - 3*2^26) * 2^-25.
__host__ __device__ inline double normal_exact(uint64_t key, uint64_t i) {
  int64_t s = 0;
  for (int j = 0; j < 6; ++j) {
    const uint64_t u = prng_u64(key, 6 * i + (uint64_t)j);
    s += (int64_t)(u >> 40) + (int64_t)((u >> 8) & 0xFFFFFFULL);
  }
  const int64_t num = 2 * s + 12 - 3 * ((int64_t)1 << 26);
  return (double)num * (1.0 / 33554432.0);
}

// ---------------------------------------------------------------------------
// wave64 helpers.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ inline float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of G consecutive lanes (G = 2, 4 or 8); every lane
// of the group receives the group sum.
template <int G>
__device__ inline float group_sum(float v) {
  static_assert(G == 2 || G == 4 || G == 8, "group size");
  v += dpp_f32<0xB1>(v);                        // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (G >= 4) v += dpp_f32<0x4E>(v);  // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (G >= 8) v += dpp_f32<0x141>(v); // row_half_mirror: other quad of the 8
  return v;
}

__device__ inline float wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ inline float wave_max(float v) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// LayerNorm of one row held by a 256-thread workgroup: the row's float4
// chunk i (columns 4 (64 i + lane) .. + 3) is v[i / 4] of wave i % 4, gamma /
// beta likewise.  The statistics are formed per lane over chunks 0 .. nch - 1
// in turn -- the mean's sum over all of them (chunks past the row hold zeros),
// the variance's over those inside the row -- exchanged through terms
// (__shared__ [4 VPW][64]), then reduced across the wave with wave_sum.  Every
// wave computes the same mean and variance and stores its own chunks.
// Products and sums stay separately rounded (no FMA contraction), so every
// kernel that restates these statistics (the skinny GEMM's LayerNorm
// prologue) reproduces them bit for bit.
template <int VPW, typename YT>
__device__ inline void ln_block_row(const float4* v, const float4* gg, const float4* bb, int wave, int lane, int N,
                                    int nch, float eps, float (*terms)[64], YT* y) {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < VPW; ++j) terms[j * 4 + wave][lane] = (v[j].x + v[j].y) + (v[j].z + v[j].w);
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nch; ++i) s += terms[i][lane];
  const float mean = wave_sum(s) / (float)N;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < VPW; ++j) {
    const float a0 = v[j].x - mean, a1 = v[j].y - mean, a2 = v[j].z - mean, a3 = v[j].w - mean;
    terms[j * 4 + wave][lane] = (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
  }
  __syncthreads();
  float q = 0.f;
  for (int i = 0; i < nch; ++i)
    if ((i * 64 + lane) * 4 < N) q += terms[i][lane];
  const float inv = rsqrtf(wave_sum(q) / (float)N + eps);
#pragma unroll
  for (int j = 0; j < VPW; ++j) {
    const int c = ((j * 4 + wave) * 64 + lane) * 4;
    if (c >= N) continue;
    const float o0 = (v[j].x - mean) * inv * gg[j].x + bb[j].x;
    const float o1 = (v[j].y - mean) * inv * gg[j].y + bb[j].y;
    const float o2 = (v[j].z - mean) * inv * gg[j].z + bb[j].z;
    const float o3 = (v[j].w - mean) * inv * gg[j].w + bb[j].w;
    if constexpr (sizeof(YT) == 4) {
      *(float4*)(y + c) = make_float4(o0, o1, o2, o3);
    } else {
      *(uint2*)(y + c) = make_uint2(pack_bf16x2(o0, o1), pack_bf16x2(o2, o3));
    }
  }
}

// layernorm_kernel's and splitk_layernorm_kernel's chunk count for a row of N
// columns (a power of two, <= 32 for N <= 8192).
__host__ __device__ inline int ln_chunks(int N) {
  int n = 1;
  while (n * 256 < N) n *= 2;
  return n;
}

constexpr float kLog2e = 1.4426950408889634f;

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace cbis

#define CBIS_REQUIRE(cond, code, ...)                  \
  do {                                                 \
    if (!(cond)) return ::cbis::fail((code), __VA_ARGS__); \
  } while (0)
