// Combine/unpermute, limited SwiGLU, and group-32 MX quantise/dequantise.
#include "glm_common.h"

namespace glm {

// out[t][c] = sum_j f32(y[inv[t*k+j]][c]) * w[t*k+j] + f32(shared[t][c])
// in the order of moe.py:198-201 (sequential j, then the shared add).
// Each thread owns 4 consecutive columns (8-byte loads of bf16).  For k <= KMAX
// the row positions and weights are loaded first, then every y row at once, so
// the kernel pays two memory latencies instead of 2k.
template <int KMAX>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t *__restrict__ y,
                                                      const int32_t *__restrict__ inv,
                                                      const float *__restrict__ w,
                                                      const uint16_t *__restrict__ shared,
                                                      const float *__restrict__ shared_parts,
                                                      int nparts, int T, int k, int d,
                                                      float *__restrict__ out) {
  // MLX forms the bf16*f32 products and their sum as separate f32 operations.
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  const int c = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (c >= d) return;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (KMAX > 0 && k <= KMAX) {
    int pos[KMAX > 0 ? KMAX : 1];
    float wj[KMAX > 0 ? KMAX : 1];
    uint2 v[KMAX > 0 ? KMAX : 1];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      pos[j] = j < k ? inv[(long long)t * k + j] : -1;
      wj[j] = j < k ? w[(long long)t * k + j] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
      if (pos[j] >= 0) v[j] = *reinterpret_cast<const uint2 *>(y + (long long)pos[j] * d + c);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (pos[j] < 0) continue;
      acc[0] = acc[0] + bf16_to_f32(v[j].x & 0xffffu) * wj[j];
      acc[1] = acc[1] + bf16_to_f32(v[j].x >> 16) * wj[j];
      acc[2] = acc[2] + bf16_to_f32(v[j].y & 0xffffu) * wj[j];
      acc[3] = acc[3] + bf16_to_f32(v[j].y >> 16) * wj[j];
    }
  } else {
    for (int j = 0; j < k; ++j) {
      const int p = inv[(long long)t * k + j];
      if (p < 0) continue;
      const float wjj = w[(long long)t * k + j];
      const uint2 vv = *reinterpret_cast<const uint2 *>(y + (long long)p * d + c);
      acc[0] = acc[0] + bf16_to_f32(vv.x & 0xffffu) * wjj;
      acc[1] = acc[1] + bf16_to_f32(vv.x >> 16) * wjj;
      acc[2] = acc[2] + bf16_to_f32(vv.y & 0xffffu) * wjj;
      acc[3] = acc[3] + bf16_to_f32(vv.y >> 16) * wjj;
    }
  }
  if (shared_parts != nullptr) {
    // shared expert output = bf16 of its K-range partial sums added in order
    float4 sp = *reinterpret_cast<const float4 *>(shared_parts + (long long)t * d + c);
    for (int q = 1; q < nparts; ++q) {
      const float4 v = *reinterpret_cast<const float4 *>(shared_parts + ((long long)q * T + t) * d + c);
      sp.x = sp.x + v.x;
      sp.y = sp.y + v.y;
      sp.z = sp.z + v.z;
      sp.w = sp.w + v.w;
    }
    acc[0] = acc[0] + bf16_round(sp.x);
    acc[1] = acc[1] + bf16_round(sp.y);
    acc[2] = acc[2] + bf16_round(sp.z);
    acc[3] = acc[3] + bf16_round(sp.w);
  } else if (shared != nullptr) {
    const uint2 v = *reinterpret_cast<const uint2 *>(shared + (long long)t * d + c);
    acc[0] = acc[0] + bf16_to_f32(v.x & 0xffffu);
    acc[1] = acc[1] + bf16_to_f32(v.x >> 16);
    acc[2] = acc[2] + bf16_to_f32(v.y & 0xffffu);
    acc[3] = acc[3] + bf16_to_f32(v.y >> 16);
  }
  *reinterpret_cast<float4 *>(out + (long long)t * d + c) = make_float4(acc[0], acc[1], acc[2], acc[3]);
}

__global__ void swiglu_kernel(const uint16_t *__restrict__ g, const uint16_t *__restrict__ u,
                              long long n, float limit, uint16_t *__restrict__ out) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    out[i] = (uint16_t)f32_to_bf16(limited_swiglu(bf16_to_f32(g[i]), bf16_to_f32(u[i]), limit));
}

// ---------------------------------------------------------------- MX codecs

// Unbiased shared exponent (clamped to [-127, 127]) for a group maximum.
// NEAREST: round(log2(amax / elem_max)) with the f32 quotient's mantissa
// compared against sqrt(2) exactly.  OCP: floor(log2(amax)) - emax_elem.
__device__ __forceinline__ int mx_exponent(float amax, float elem_max, int emax_elem, int rule) {
  if (!(amax <= 3.402823466e38f)) return 128;  // inf/NaN -> scale byte 255
  if (amax == 0.0f) return -127;
  int n;
  if (rule == GLM_MX_RULE_NEAREST) {
    const float s = __fdiv_rn(amax, elem_max);
    const uint32_t bits = __float_as_uint(s);
    const int biased = (bits >> 23) & 0xff;
    if (biased == 0) {
      // subnormal quotient: normalise the mantissa
      uint32_t m = bits & 0x7fffffu;
      int ex = -126;
      while (!(m & 0x800000u)) {
        m <<= 1;
        --ex;
      }
      n = ex + (((m & 0x7fffffu) | 0x3f800000u) > 0x3fb504f3u ? 1 : 0);
    } else {
      n = biased - 127 + (((bits & 0x7fffffu) | 0x3f800000u) > 0x3fb504f3u ? 1 : 0);
    }
  } else {
    const uint32_t bits = __float_as_uint(amax);
    int biased = (bits >> 23) & 0xff;
    int ex;
    if (biased == 0) {
      uint32_t m = bits & 0x7fffffu;
      ex = -126;
      while (!(m & 0x800000u)) {
        m <<= 1;
        --ex;
      }
    } else {
      ex = biased - 127;
    }
    n = ex - emax_elem;
  }
  return n < -127 ? -127 : (n > 127 ? 127 : n);
}

// |v| (already divided by the group scale) -> E4M3FN magnitude code, RNE,
// saturating at 448 (code 0x7e).
__device__ __forceinline__ uint32_t e4m3_code(float a) {
  a = fminf(a, 448.0f);
  if (a < 0.015625f) {  // below 2^-6: subnormal grid of 2^-9
    const float r = a * 512.0f;  // exact
    float n = rintf(r);           // ties to even
    return (uint32_t)n;           // 0..8 (8 == 2^-6, first normal, code 0x08)
  }
  const uint32_t bits = __float_as_uint(a);
  const int ex = (int)((bits >> 23) & 0xff) - 127;  // -6..8
  // keep 3 mantissa bits with round-to-nearest-even on the f32 pattern
  uint32_t m = bits & 0x7fffffu;
  const uint32_t keep = m >> 20;
  const uint32_t rest = m & 0xfffffu;
  uint32_t q = ((uint32_t)(ex + 7) << 3) | keep;
  if (rest > 0x80000u || (rest == 0x80000u && (keep & 1))) q += 1;  // may carry into exponent
  return q > 0x7eu ? 0x7eu : q;
}

// |v| -> E2M1 magnitude code (0..7), RNE, saturating at 6.
__device__ __forceinline__ uint32_t e2m1_code(float a) {
  a = fminf(a, 6.0f);
  // thresholds between 0,.5,1,1.5,2,3,4,6; ties go to the even code
  if (a < 0.25f) return 0;
  if (a == 0.25f) return 0;
  if (a < 0.75f) return 1;
  if (a == 0.75f) return 2;
  if (a < 1.25f) return 2;
  if (a == 1.25f) return 2;
  if (a < 1.75f) return 3;
  if (a == 1.75f) return 4;
  if (a < 2.5f) return 4;
  if (a == 2.5f) return 4;
  if (a < 3.5f) return 5;
  if (a == 3.5f) return 6;
  if (a < 5.0f) return 6;
  if (a == 5.0f) return 6;
  return 7;
}

// One thread per 32-element group.
__global__ void mx_quantize_kernel(const uint16_t *__restrict__ w, long long groups, int fmt,
                                   int rule, uint8_t *__restrict__ codes,
                                   uint8_t *__restrict__ scales) {
  for (long long gi = blockIdx.x * (long long)blockDim.x + threadIdx.x; gi < groups;
       gi += (long long)gridDim.x * blockDim.x) {
    const uint16_t *src = w + gi * 32;
    float v[32];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      v[i] = bf16_to_f32(src[i]);
      amax = fmaxf(amax, fabsf(v[i]));
    }
    const bool is8 = fmt == GLM_FMT_MXFP8;
    const int ex = mx_exponent(amax, is8 ? 448.0f : 6.0f, is8 ? 8 : 2, rule);
    scales[gi] = (uint8_t)(ex + 127);
    const float inv = ldexpf(1.0f, -ex);  // exact power of two
    if (is8) {
      uint8_t *dst = codes + gi * 32;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const float sv = v[i] * inv;
        uint32_t c = e4m3_code(fabsf(sv));
        if (__float_as_uint(sv) >> 31) c |= 0x80u;
        dst[i] = (uint8_t)c;
      }
    } else {
      uint8_t *dst = codes + gi * 16;
#pragma unroll
      for (int i = 0; i < 32; i += 2) {
        const float s0 = v[i] * inv, s1 = v[i + 1] * inv;
        uint32_t c0 = e2m1_code(fabsf(s0)) | ((__float_as_uint(s0) >> 31) << 3);
        uint32_t c1 = e2m1_code(fabsf(s1)) | ((__float_as_uint(s1) >> 31) << 3);
        dst[i >> 1] = (uint8_t)(c0 | (c1 << 4));
      }
    }
  }
}

// Dequantisation through the same hardware converts the MFMA kernels use.
__global__ void mx_dequantize_kernel(const uint8_t *__restrict__ codes,
                                     const uint8_t *__restrict__ scales, long long groups,
                                     int fmt, float *__restrict__ out) {
  for (long long gi = blockIdx.x * (long long)blockDim.x + threadIdx.x; gi < groups;
       gi += (long long)gridDim.x * blockDim.x) {
    const float sc = e8m0_to_f32(scales[gi]);
    float *dst = out + gi * 32;
    if (fmt == GLM_FMT_MXFP4) {
      const uint32_t *src = reinterpret_cast<const uint32_t *>(codes + gi * 16);
#pragma unroll
      for (int wdx = 0; wdx < 4; ++wdx) {
        const glm_bf16x8 v = mxfp4_word_to_bf16x8(src[wdx], sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) dst[wdx * 8 + i] = (float)v[i];
      }
    } else {
      const uint32_t *src = reinterpret_cast<const uint32_t *>(codes + gi * 32);
#pragma unroll
      for (int wdx = 0; wdx < 8; wdx += 2) {
        const glm_bf16x8 v = mxfp8_words_to_bf16x8(src[wdx], src[wdx + 1], sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) dst[wdx * 4 + i] = (float)v[i];
      }
    }
  }
}

}  // namespace glm

int glm_combine_parts_launch(hipStream_t stream, const uint16_t *y, const int32_t *inv,
                             const float *w, const uint16_t *shared, const float *shared_parts,
                             int nparts, int T, int k, int d, float *out) {
  if (T == 0) return GLM_OK;
  dim3 grid((d / 4 + 255) / 256, T);
  if (k <= 8)
    hipLaunchKernelGGL(glm::combine_kernel<8>, grid, dim3(256), 0, stream, y, inv, w, shared,
                       shared_parts, nparts, T, k, d, out);
  else if (k <= 16)
    hipLaunchKernelGGL(glm::combine_kernel<16>, grid, dim3(256), 0, stream, y, inv, w, shared,
                       shared_parts, nparts, T, k, d, out);
  else
    hipLaunchKernelGGL(glm::combine_kernel<0>, grid, dim3(256), 0, stream, y, inv, w, shared,
                       shared_parts, nparts, T, k, d, out);
  GLM_LAUNCH_CHECK("combine_kernel");
  return GLM_OK;
}

int glm_combine_launch(hipStream_t stream, const uint16_t *y, const int32_t *inv, const float *w,
                       const uint16_t *shared, int T, int k, int d, float *out) {
  return glm_combine_parts_launch(stream, y, inv, w, shared, nullptr, 0, T, k, d, out);
}

static int grid_for(long long n, int block) {
  long long g = (n + block - 1) / block;
  return (int)(g > 65536 ? 65536 : (g < 1 ? 1 : g));
}

extern "C" int glm_moe_combine(void *stream, const uint16_t *y, const int32_t *inv,
                               const float *weights, const uint16_t *shared, int T, int top_k,
                               int d, float *out) {
  glm::clear_error();
  GLM_REQUIRE(y && inv && weights && out, GLM_ERR_INVALID_ARGUMENT,
              "combine: null pointer argument");
  GLM_REQUIRE(T >= 0 && top_k >= 1 && d > 0, GLM_ERR_INVALID_ARGUMENT, "combine: invalid sizes");
  GLM_REQUIRE(d % 4 == 0, GLM_ERR_UNSUPPORTED_SHAPE, "combine: d=%d not a multiple of 4", d);
  GLM_REQUIRE(glm_aligned16({y, out, shared}), GLM_ERR_INVALID_ARGUMENT,
              "combine: buffers must be 16-byte aligned");
  return glm_combine_launch((hipStream_t)stream, y, inv, weights, shared, T, top_k, d, out);
}

extern "C" int glm_limited_swiglu(void *stream, const uint16_t *gate, const uint16_t *up,
                                  int64_t n, float limit, uint16_t *out) {
  glm::clear_error();
  GLM_REQUIRE(gate && up && out, GLM_ERR_INVALID_ARGUMENT, "limited_swiglu: null pointer");
  GLM_REQUIRE(n >= 0, GLM_ERR_INVALID_ARGUMENT, "limited_swiglu: negative size");
  if (n == 0) return GLM_OK;
  hipLaunchKernelGGL(glm::swiglu_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                     (hipStream_t)stream, gate, up, (long long)n, glm_limit_bf16(limit), out);
  GLM_LAUNCH_CHECK("swiglu_kernel");
  return GLM_OK;
}

extern "C" int glm_mx_quantize(void *stream, const uint16_t *w, int rows, int cols, int fmt,
                               int rule, uint8_t *codes, uint8_t *scales) {
  glm::clear_error();
  GLM_REQUIRE(w && codes && scales, GLM_ERR_INVALID_ARGUMENT, "mx_quantize: null pointer");
  GLM_REQUIRE(fmt == GLM_FMT_MXFP8 || fmt == GLM_FMT_MXFP4, GLM_ERR_INVALID_ARGUMENT,
              "mx_quantize: unsupported format %d", fmt);
  GLM_REQUIRE(rule == GLM_MX_RULE_NEAREST || rule == GLM_MX_RULE_OCP, GLM_ERR_INVALID_ARGUMENT,
              "mx_quantize: unknown scale rule %d", rule);
  GLM_REQUIRE(rows >= 0 && cols > 0, GLM_ERR_INVALID_ARGUMENT, "mx_quantize: invalid shape");
  GLM_REQUIRE(cols % 32 == 0, GLM_ERR_UNSUPPORTED_SHAPE,
              "mx_quantize: group-32 needs cols %% 32 == 0, got %d", cols);
  const long long groups = (long long)rows * (cols / 32);
  if (groups == 0) return GLM_OK;
  hipLaunchKernelGGL(glm::mx_quantize_kernel, dim3(grid_for(groups, 256)), dim3(256), 0,
                     (hipStream_t)stream, w, groups, fmt, rule, codes, scales);
  GLM_LAUNCH_CHECK("mx_quantize_kernel");
  return GLM_OK;
}

extern "C" int glm_mx_dequantize(void *stream, const uint8_t *codes, const uint8_t *scales,
                                 int rows, int cols, int fmt, float *out) {
  glm::clear_error();
  GLM_REQUIRE(codes && scales && out, GLM_ERR_INVALID_ARGUMENT, "mx_dequantize: null pointer");
  GLM_REQUIRE(fmt == GLM_FMT_MXFP8 || fmt == GLM_FMT_MXFP4, GLM_ERR_INVALID_ARGUMENT,
              "mx_dequantize: unsupported format %d", fmt);
  GLM_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, GLM_ERR_UNSUPPORTED_SHAPE,
              "mx_dequantize: invalid shape %d x %d", rows, cols);
  GLM_REQUIRE(glm_aligned16({codes}), GLM_ERR_INVALID_ARGUMENT,
              "mx_dequantize: codes must be 16-byte aligned");
  const long long groups = (long long)rows * (cols / 32);
  if (groups == 0) return GLM_OK;
  hipLaunchKernelGGL(glm::mx_dequantize_kernel, dim3(grid_for(groups, 256)), dim3(256), 0,
                     (hipStream_t)stream, codes, scales, groups, fmt, out);
  GLM_LAUNCH_CHECK("mx_dequantize_kernel");
  return GLM_OK;
}
