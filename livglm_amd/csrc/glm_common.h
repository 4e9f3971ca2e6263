// Shared device helpers and host-side error plumbing for libglm53moe.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <initializer_list>

#include "glm53_moe.h"

// ---------------------------------------------------------------- host errors

namespace glm {

void set_error(const char *fmt, ...);
void clear_error();

// hyper_residual of the decoder FFN site, fused into the MoE layer's last
// kernel (glm_moe_forward_hc): out[t][j] = post[t][j] y[t] + sum_i comb[t][i][j] res[t][i]
struct HcFuse {
  const float *res, *post, *comb;  // [T][hc][d], [T][hc], [T][hc][hc]
  float *out;                      // [T][hc][d]
  int hc, bf16;                    // bf16: GLM_HC_BF16_STREAMS rounding points
};

}  // namespace glm

#define GLM_REQUIRE(cond, code, ...)  \
  do {                                \
    if (!(cond)) {                    \
      glm::set_error(__VA_ARGS__);    \
      return (code);                  \
    }                                 \
  } while (0)

#define GLM_HIP_CHECK(expr)                                                              \
  do {                                                                                   \
    hipError_t glm_err_ = (expr);                                                        \
    if (glm_err_ != hipSuccess) {                                                        \
      glm::set_error("%s failed: %s", #expr, hipGetErrorString(glm_err_));              \
      return GLM_ERR_HIP;                                                                \
    }                                                                                    \
  } while (0)

// Check the launch that was just enqueued.
#define GLM_LAUNCH_CHECK(name)                                                           \
  do {                                                                                   \
    hipError_t glm_err_ = hipGetLastError();                                             \
    if (glm_err_ != hipSuccess) {                                                        \
      glm::set_error("launch of %s failed: %s", name, hipGetErrorString(glm_err_));     \
      return GLM_ERR_HIP;                                                                \
    }                                                                                    \
  } while (0)

// True when every non-null pointer is 16-byte aligned (the kernels use
// 128-bit loads and stores).
static inline bool glm_aligned16(std::initializer_list<const void *> ptrs) {
  for (const void *p : ptrs)
    if (p != nullptr && (reinterpret_cast<uintptr_t>(p) & 15u) != 0) return false;
  return true;
}

// ---------------------------------------------------------------- device types

typedef __attribute__((ext_vector_type(8))) __bf16 glm_bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 glm_bf16x2;
typedef __attribute__((ext_vector_type(4))) float glm_f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t glm_u32x4;

namespace glm {

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// f32 -> bf16 bits, round to nearest even (gfx950's v_cvt_pk_bf16_f32;
// subnormals are kept, NaN becomes a quiet NaN).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Element i of the router weights w [n] split into three bf16 parts
// (w = p0 + p1 + p2: p0 = bf16(w), p1 = bf16(w - p0), p2 = bf16(w - p0 - p1)),
// stored at ws[i], ws[n + i], ws[2 n + i].
__device__ __forceinline__ void bf16x3_split_one(const float *__restrict__ w, long long n,
                                                 uint16_t *__restrict__ ws, long long i) {
  const float v = w[i];
  const uint32_t b0 = f32_to_bf16(v);
  const float r1 = v - bf16_to_f32(b0);
  const uint32_t b1 = f32_to_bf16(r1);
  const float r2 = r1 - bf16_to_f32(b1);
  ws[i] = (uint16_t)b0;
  ws[n + i] = (uint16_t)b1;
  ws[2 * n + i] = (uint16_t)f32_to_bf16(r2);
}

// E8M0 byte -> f32 scale 2^(e-127) (byte 255 = NaN).
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  // branch-free: two selects on the shifted exponent
  uint32_t u = e << 23;
  u = e == 0u ? 0x00400000u : u;    // 2^-127, subnormal
  u = e == 255u ? 0x7fc00000u : u;  // NaN
  return __uint_as_float(u);
}

// sigmoid in f32: y = 1/(1+exp(|x|)); x<0 ? y : 1-y.
__device__ __forceinline__ float sigmoid_f32(float x) {
  float y = 1.0f / (1.0f + expf(fabsf(x)));
  return x < 0.0f ? y : 1.0f - y;
}

// The bank keeps an MXFP4 matrix of `rows` x K codes (K / 2 bytes a row in
// the checkpoint) tile-major when rows % 16 == 0 and K % 128 == 0 -- every
// geometry the MFMA kernels take; any other matrix stays row-major.  Tile
// t (rows 16t..16t+15) and chunk c (codes 128c..128c+127) form the 1 KB
// block at byte (t K/128 + c) * 1024, whose 16-byte piece l = r + 16 q holds
// row 16t + r, codes 128c + 32q .. +31 (one E8M0 group): a wave's 64 lanes
// read one block as 1 KB of contiguous memory.  Piece p (bytes 16p..16p+15)
// of a row-major row goes to piece mxfp4_tile_piece(row, p, K).
__host__ __device__ inline bool mxfp4_tiled(long long rows, long long K) {
  return rows % 16 == 0 && K % 128 == 0;
}
__host__ __device__ inline long long mxfp4_tile_piece(long long row, long long p, long long K) {
  return ((row >> 4) * (K / 128) + (p >> 2)) * 64 + (row & 15) + 16 * (p & 3);
}

// limited_swiglu on one element with bf16 intermediates (expert_ssd.py:103-107):
// g = min(g, L); u = clip(u, -L, L); h = bf16(bf16(g * bf16(sigmoid(g))) * u).
// The clamps are IEEE minimum / maximum, so a NaN g or u passes through them,
// as through mx.minimum / mx.clip.
__device__ __forceinline__ float limited_swiglu(float g, float u, float limit_bf16) {
  if (limit_bf16 > 0.0f) {
    g = __builtin_elementwise_minimum(g, limit_bf16);
    u = __builtin_elementwise_maximum(__builtin_elementwise_minimum(u, limit_bf16), -limit_bf16);
  }
  float s = bf16_round(sigmoid_f32(g));
  float a = bf16_round(g * s);
  return bf16_round(a * u);
}

// Two f32 -> bf16 roundings (nearest even) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ void bf16_round2(float &a, float &b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
  a = __uint_as_float(p << 16);
  b = __uint_as_float(p & 0xffff0000u);
}

// limited_swiglu on two elements with bf16 intermediates (expert_ssd.py:
// 103-107), for the epilogues of the many-token GEMMs: g, u the bf16 gate and
// up values; lim the bf16 limit, or +inf when there is none (NaN passes
// through the clamps, IEEE minimum / maximum, as it does through the
// reference's).  The sigmoid is
// 1 / (1 + 2^(-g log2 e)) on the hardware exp2 and reciprocal: within a few
// f32 ulp of sigmoid_f32, which the bf16 rounding that follows absorbs except
// within a few ulp of a bf16 rounding tie.  Each bf16 rounding of the pair
// is one convert.
__device__ __forceinline__ void limited_swiglu2_fast(float g0, float g1, float u0, float u1,
                                                     float lim, float &h0, float &h1) {
  g0 = __builtin_elementwise_minimum(g0, lim);
  g1 = __builtin_elementwise_minimum(g1, lim);
  u0 = __builtin_elementwise_maximum(__builtin_elementwise_minimum(u0, lim), -lim);
  u1 = __builtin_elementwise_maximum(__builtin_elementwise_minimum(u1, lim), -lim);
  float s0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g0 * -1.44269504088896341f));
  float s1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g1 * -1.44269504088896341f));
  bf16_round2(s0, s1);
  float a0 = g0 * s0, a1 = g1 * s1;
  bf16_round2(a0, a1);
  h0 = a0 * u0;
  h1 = a1 * u1;
  bf16_round2(h0, h1);
}

// 8 packed E2M1 codes (one u32, low nibble first) -> 8 bf16 times `scale`,
// through the gfx950 scaled converts (exact: every value fits bf16).
__device__ __forceinline__ glm_bf16x8 mxfp4_word_to_bf16x8(uint32_t w, float scale) {
  const glm_bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  const glm_bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  const glm_bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  const glm_bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  glm_bf16x8 o;
  o[0] = p0[0];
  o[1] = p0[1];
  o[2] = p1[0];
  o[3] = p1[1];
  o[4] = p2[0];
  o[5] = p2[1];
  o[6] = p3[0];
  o[7] = p3[1];
  return o;
}

// 8 E4M3FN codes (two u32, byte 0 first) -> 8 bf16 times `scale`.
__device__ __forceinline__ glm_bf16x8 mxfp8_words_to_bf16x8(uint32_t w0, uint32_t w1,
                                                            float scale) {
  const glm_bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, false);
  const glm_bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, true);
  const glm_bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, false);
  const glm_bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, true);
  glm_bf16x8 o;
  o[0] = p0[0];
  o[1] = p0[1];
  o[2] = p1[0];
  o[3] = p1[1];
  o[4] = p2[0];
  o[5] = p2[1];
  o[6] = p3[0];
  o[7] = p3[1];
  return o;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

}  // namespace glm

// Host helper: the swiglu limit as the bf16 value MLX compares against.
static inline float glm_limit_bf16(float limit) {
  union {
    float f;
    uint32_t u;
  } v;
  v.f = limit;
  uint32_t u = v.u;
  u += 0x7fffu + ((u >> 16) & 1u);
  v.u = (u >> 16) << 16;
  return v.f;
}
