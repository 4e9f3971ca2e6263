// The FFN site of a GLM-5.3-Flash decoder layer around the routed-MoE layer
// (model.py:132-136):
//
//   post, comb, collapsed = ffn_hc(streams)           HyperConnection, mhc.py:23-48
//   y = mlp(post_attention_layernorm(collapsed))      RMSNorm (layers.py:119-131) + MoE
//   out = hyper_residual(streams, y, post, comb)      mhc.py:51-60
//
// streams are the hc residual streams of a token, f32 [T][hc][d].  The
// HyperConnection is a two-row (T-row) GEMV of the unweighted-RMS-normalised
// flattened streams against fn [2 hc + hc^2][hc d] followed by a few dozen
// scalars per token (sigmoid gates, a row softmax and Sinkhorn normalisation of
// the hc x hc mixing matrix), then a pre-weighted sum of the streams.  Here:
//
//   hc_mix_kernel     K-sliced GEMV: one workgroup per 256 columns of hc d and
//                     four tokens, fn read once per token group; per-slice
//                     partial dot products and sums of squares to a workspace.
//   hc_finish_kernel  one workgroup per token: partials summed in slice order,
//                     the gate/mixing scalars on one wave through LDS, the
//                     collapsed stream, and (optionally) the post-attention
//                     RMSNorm with its bf16 cast, the MoE layer's input.
//   hc_post_kernel    hyper_residual: out[j] = post[j] y + sum_i comb[i][j] res[i].
//   rms_norm_kernel   standalone RMSNorm (weighted or not), f32 and/or bf16 out.
#include "glm_common.h"
#include "topk_select.h"  // wave_lds_sync

// Every product and sum is rounded on its own, as the reference's separate
// array operations are (no fused multiply-add).
#pragma clang fp contract(off)

namespace glm {

constexpr int kHcThreads = 256;
constexpr int kHcSlice = 256;        // columns of hc*d per hc_mix chunk
constexpr int kHcMaxSlices = 64;     // hc_mix workgroups along K (chunks beyond loop)
constexpr int kHcTokens = 4;         // tokens per hc_mix workgroup
constexpr int kHcMaxMult = 8;        // hc <= 8: M = 2 hc + hc^2 <= 80
constexpr int kHcMaxM = 2 * kHcMaxMult + kHcMaxMult * kHcMaxMult;
constexpr int kHcMaxD = 8192;        // collapsed row kept in LDS (32 KB)

__device__ __forceinline__ void lds_sync() { __syncthreads(); }

// Sum over a 256-thread workgroup in a fixed order (wave butterflies, then
// waves 0..3 in order); every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  lds_sync();
  const float s = (red[0] + red[1]) + (red[2] + red[3]);
  lds_sync();
  return s;
}

// partial[s][t][m] = sum over the columns of workgroup s of x[t][k] fn[m][k]
// (m < M); partial[s][t][M] = the sum of x[t][k]^2 over them.  Workgroup s
// takes the 256-column chunks s, s + S, ... of the K = hc d columns; wave w
// owns the rows w, w + 4, ... (ROWS at most).  Every load of a chunk -- the
// token rows and all of the wave's fn rows -- is issued before any product,
// and lanes keep running sums, so a workgroup waits on memory once per chunk
// and reduces across lanes once at the end.
template <int ROWS>
__global__ __launch_bounds__(kHcThreads) void hc_mix_kernel(const float *x, const float *fn, int T,
                                                            int K, int M, float *partial) {
  const int s = blockIdx.x, S = gridDim.x;
  const int t0 = blockIdx.y * kHcTokens;
  const int nt = min(kHcTokens, T - t0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nchunks = (K + kHcSlice - 1) / kHcSlice;
  float acc[ROWS][kHcTokens], sq[kHcTokens];
#pragma unroll
  for (int t = 0; t < kHcTokens; ++t) {
    sq[t] = 0.f;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r][t] = 0.f;
  }
  for (int c = s; c < nchunks; c += S) {
    const int k = c * kHcSlice + 4 * lane;
    const bool in = k < K;  // K % 4 == 0: a lane's 4 columns are all in or all out
    glm_f32x4 xv[kHcTokens], w[ROWS];
#pragma unroll
    for (int t = 0; t < kHcTokens; ++t) {
      xv[t] = glm_f32x4{0.f, 0.f, 0.f, 0.f};
      if (t < nt && in)
        xv[t] = *reinterpret_cast<const glm_f32x4 *>(x + (size_t)(t0 + t) * K + k);
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const int m = wave + 4 * r;
      w[r] = glm_f32x4{0.f, 0.f, 0.f, 0.f};
      if (m < M && in) w[r] = *reinterpret_cast<const glm_f32x4 *>(fn + (size_t)m * K + k);
    }
#pragma unroll
    for (int t = 0; t < kHcTokens; ++t) {
      sq[t] += xv[t][0] * xv[t][0] + xv[t][1] * xv[t][1] + xv[t][2] * xv[t][2] +
               xv[t][3] * xv[t][3];
#pragma unroll
      for (int r = 0; r < ROWS; ++r)
        acc[r][t] += xv[t][0] * w[r][0] + xv[t][1] * w[r][1] + xv[t][2] * w[r][2] +
                     xv[t][3] * w[r][3];
    }
  }
#pragma unroll
  for (int t = 0; t < kHcTokens; ++t) {
    if (t >= nt) break;  // uniform
    float *out = partial + ((size_t)s * T + t0 + t) * (M + 1);
    if (wave == 0) {
      const float q = wave_sum(sq[t]);
      if (lane == 0) out[M] = q;
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const int m = wave + 4 * r;
      if (m >= M) break;  // uniform
      const float p = wave_sum(acc[r][t]);
      if (lane == 0) out[m] = p;
    }
  }
}

// A gate logit as the reference forms it: (mixed * inv_rms) * scale + base
// (mhc.py:38-41).
__device__ __forceinline__ float gate_logit(float raw, float inv, float scale, float base) {
  return raw * inv * scale + base;
}

struct HcFinishArgs {
  const float *streams;  // [T][hc][d]
  const float *partial;  // [S][T][M + 1]
  const float *base, *scale;
  const float *norm_weight;  // [d] or nullptr (unweighted)
  int T, hc, d, S, iters;
  int bf16_streams;  // GLM_HC_BF16_STREAMS: collapsed is rounded to bf16 (the streams' dtype)
  float rms_eps, hc_eps, norm_eps;
  float *post, *comb, *collapsed;  // [T][hc], [T][hc][hc], [T][d] (collapsed may be null)
  uint16_t *normed;                // bf16 [T][d] or nullptr
};

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(dpp_i32<CTRL>(__float_as_int(v)));
}

// Sums and maxima over the hc x hc mixing matrix held one entry per lane
// (lane = i hc + j, lanes >= hc^2 idle).  hc = 2, 4: DPP lane moves within a
// row of 16 lanes (quad swaps along a matrix row, row rotations by 8 then 4
// down a column of hc = 4); hc = 8: xor shuffles; other hc: through LDS in
// ascending order.  Every lane of a row (column) ends with the same value.
struct HcMatrix {
  enum Mode { kDpp, kShuffle, kLds };
  int hc;
  Mode mode;
  bool mine;
  int i, j, lane;
  float *lds;  // hc^2 floats

  __device__ static float op(float a, float b, bool max) { return max ? fmaxf(a, b) : a + b; }

  __device__ float row_reduce(float v, bool max) const {
    if (mode == kDpp) {
      if (hc >= 2) v = op(v, dpp_f32<0xB1>(v), max);  // quad_perm [1,0,3,2]: column j ^ 1
      if (hc == 4) v = op(v, dpp_f32<0x4E>(v), max);  // quad_perm [2,3,0,1]: column j ^ 2
      return v;
    }
    if (mode == kShuffle) {
      for (int off = 1; off < hc; off <<= 1) v = op(v, __shfl_xor(v, off), max);
      return v;
    }
    wave_lds_sync();
    if (mine) lds[lane] = v;
    wave_lds_sync();
    if (!mine) return v;
    float r = lds[i * hc];
    for (int q = 1; q < hc; ++q) r = op(r, lds[i * hc + q], max);
    return r;
  }

  __device__ float col_sum(float v) const {
    if (mode == kDpp) {
      if (hc == 2) v += dpp_f32<0x4E>(v);  // row i ^ 1 (lanes two apart)
      if (hc == 4) {
        v += dpp_f32<0x128>(v);  // row_ror:8: rows i and i ^ 2
        v += dpp_f32<0x124>(v);  // row_ror:4: the other pair
      }
      return v;
    }
    if (mode == kShuffle) {
      for (int off = hc; off < hc * hc; off <<= 1) v += __shfl_xor(v, off);
      return v;
    }
    wave_lds_sync();
    if (mine) lds[lane] = v;
    wave_lds_sync();
    if (!mine) return v;
    float r = lds[j];
    for (int q = 1; q < hc; ++q) r += lds[q * hc + j];
    return r;
  }
};

__global__ __launch_bounds__(kHcThreads) void hc_finish_kernel(HcFinishArgs a) {
  __shared__ float pbuf[kHcMaxSlices * (kHcMaxM + 1)];
  __shared__ float mixed[kHcMaxM + 1];
  __shared__ float cm[kHcMaxMult * kHcMaxMult];
  __shared__ float pre[kHcMaxMult];
  __shared__ float red[4];
  extern __shared__ float row[];  // collapsed row, d floats
  const int t = blockIdx.x;
  const int hc = a.hc, d = a.d, M = 2 * hc + hc * hc;
  const int K = hc * d;
  const int tid = threadIdx.x;
  // the first pass of the collapsed sum reads its streams now: they do not
  // depend on the gates, so their latency hides behind everything before it
  const float *st = a.streams + (size_t)t * K;
  glm_f32x4 sv[2][kHcMaxMult];
  auto load_streams = [&](int c0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = c0 + u * 4 * kHcThreads;
#pragma unroll
      for (int i = 0; i < kHcMaxMult; ++i)
        if (i < hc && c < d) sv[u][i] = *reinterpret_cast<const glm_f32x4 *>(st + (size_t)i * d + c);
    }
  };
  load_streams(4 * tid);
  // the per-workgroup partials of hc_mix: all loads issued together, then
  // summed in workgroup order from LDS
  const int n = a.S * (M + 1);
  for (int q0 = tid; q0 < n; q0 += 4 * kHcThreads) {
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int q = q0 + u * kHcThreads;
      v[u] = 0.f;
      if (q < n) v[u] = a.partial[((size_t)(q / (M + 1)) * a.T + t) * (M + 1) + q % (M + 1)];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (q0 + u * kHcThreads < n) pbuf[q0 + u * kHcThreads] = v[u];
  }
  lds_sync();
  if (tid <= M) {
    float acc = 0.f;
    for (int s = 0; s < a.S; ++s) acc += pbuf[s * (M + 1) + tid];
    mixed[tid] = acc;
  }
  lds_sync();
  if (tid < 64) {
    // flat = streams * inv_rms, mixed = flat @ fn^T = inv_rms * (streams @ fn^T)
    const float inv = 1.0f / sqrtf(mixed[M] / (float)K + a.rms_eps);
    const int lane = tid;
    const HcMatrix::Mode mode = hc <= 2 || hc == 4 ? HcMatrix::kDpp
                                : hc == 8            ? HcMatrix::kShuffle
                                                     : HcMatrix::kLds;
    const HcMatrix mat{hc, mode, lane < hc * hc, lane / hc, lane % hc, lane, cm};
    if (lane < hc) {
      const float p = sigmoid_f32(gate_logit(mixed[lane], inv, a.scale[0], a.base[lane])) +
                      a.hc_eps;
      pre[lane] = p;
      a.post[(size_t)t * hc + lane] =
          2.0f * sigmoid_f32(gate_logit(mixed[hc + lane], inv, a.scale[1], a.base[hc + lane]));
    }
    float c = 0.f;
    if (mat.mine) c = gate_logit(mixed[2 * hc + lane], inv, a.scale[2], a.base[2 * hc + lane]);
    // row softmax (mhc.py:41) + eps, the column normalisation, then
    // iters - 1 rounds of (row, column) normalisation (mhc.py:42-45)
    const float mx = mat.row_reduce(c, true);
    c = expf(c - mx);
    c = c / mat.row_reduce(c, false) + a.hc_eps;
    c = c / (mat.col_sum(c) + a.hc_eps);
    for (int it = 1; it < a.iters; ++it) {
      c = c / (mat.row_reduce(c, false) + a.hc_eps);
      c = c / (mat.col_sum(c) + a.hc_eps);
    }
    if (mat.mine) a.comb[(size_t)t * hc * hc + lane] = c;
  }
  lds_sync();
  // collapsed[c] = sum_i pre[i] streams[t][i][c] (i ascending); two column
  // groups per pass with all their stream loads issued together
  float sq = 0.f;
  for (int c0 = 4 * tid; c0 < d; c0 += 8 * kHcThreads) {
    if (c0 != 4 * tid) load_streams(c0);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = c0 + u * 4 * kHcThreads;
      if (c >= d) break;
      glm_f32x4 v = glm_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < kHcMaxMult; ++i) {
        if (i < hc) {
          const float p = pre[i];
          v = glm_f32x4{v[0] + p * sv[u][i][0], v[1] + p * sv[u][i][1], v[2] + p * sv[u][i][2],
                        v[3] + p * sv[u][i][3]};
        }
      }
      if (a.bf16_streams)
        v = glm_f32x4{bf16_round(v[0]), bf16_round(v[1]), bf16_round(v[2]), bf16_round(v[3])};
      *reinterpret_cast<glm_f32x4 *>(row + c) = v;
      if (a.collapsed) *reinterpret_cast<glm_f32x4 *>(a.collapsed + (size_t)t * d + c) = v;
      sq += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
  }
  if (a.normed == nullptr) return;
  // post-attention RMSNorm of the collapsed row, rounded to bf16
  const float total = block_sum(sq, red);
  const float inv = 1.0f / sqrtf(total / (float)d + a.norm_eps);
  for (int c = 4 * tid; c < d; c += 4 * kHcThreads) {
    const glm_f32x4 v = *reinterpret_cast<const glm_f32x4 *>(row + c);
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float r = v[q] * inv;
      if (a.norm_weight) r *= a.norm_weight[c + q];
      o[q] = f32_to_bf16(r);
    }
    *reinterpret_cast<uint2 *>(a.normed + (size_t)t * d + c) =
        uint2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
  }
}

// out[t][j][c] = post[t][j] y[t][c] + sum_i comb[t][i][j] residual[t][i][c]; with
// bf16 streams (BF16 = true) post and comb are rounded to bf16 and the mixing
// sum is rounded to bf16 before the f32 add (mhc.py:57-59 in the streams' dtype).
template <bool BF16>
__global__ __launch_bounds__(kHcThreads) void hc_post_kernel(const float *res, const float *y,
                                                             const float *post, const float *comb,
                                                             int hc, int d, float *out) {
  const int t = blockIdx.y;
  const int c = 4 * (blockIdx.x * kHcThreads + threadIdx.x);
  if (c >= d) return;
  const float *r = res + (size_t)t * hc * d;
  glm_f32x4 rv[kHcMaxMult];
#pragma unroll
  for (int i = 0; i < kHcMaxMult; ++i)
    if (i < hc) rv[i] = *reinterpret_cast<const glm_f32x4 *>(r + (size_t)i * d + c);
  const glm_f32x4 yv = *reinterpret_cast<const glm_f32x4 *>(y + (size_t)t * d + c);
  for (int j = 0; j < hc; ++j) {
    float pj = post[(size_t)t * hc + j];
    if (BF16) pj = bf16_round(pj);
    glm_f32x4 m = glm_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kHcMaxMult; ++i) {
      if (i < hc) {
        float w = comb[((size_t)t * hc + i) * hc + j];
        if (BF16) w = bf16_round(w);
        m = glm_f32x4{m[0] + w * rv[i][0], m[1] + w * rv[i][1], m[2] + w * rv[i][2],
                      m[3] + w * rv[i][3]};
      }
    }
    if (BF16) m = glm_f32x4{bf16_round(m[0]), bf16_round(m[1]), bf16_round(m[2]), bf16_round(m[3])};
    const glm_f32x4 o = glm_f32x4{pj * yv[0] + m[0], pj * yv[1] + m[1], pj * yv[2] + m[2],
                                  pj * yv[3] + m[3]};
    *reinterpret_cast<glm_f32x4 *>(out + ((size_t)t * hc + j) * d + c) = o;
  }
}

__global__ __launch_bounds__(kHcThreads) void rms_norm_kernel(const float *x, int d,
                                                              const float *weight, float eps,
                                                              float *out, uint16_t *out_bf16) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const float *xr = x + (size_t)t * d;
  float sq = 0.f;
  for (int c = 4 * threadIdx.x; c < d; c += 4 * kHcThreads) {
    const glm_f32x4 v = *reinterpret_cast<const glm_f32x4 *>(xr + c);
    sq += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  }
  const float inv = 1.0f / sqrtf(block_sum(sq, red) / (float)d + eps);
  for (int c = 4 * threadIdx.x; c < d; c += 4 * kHcThreads) {
    const glm_f32x4 v = *reinterpret_cast<const glm_f32x4 *>(xr + c);
    glm_f32x4 r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      r[q] = v[q] * inv;
      if (weight) r[q] *= weight[c + q];
    }
    if (out) *reinterpret_cast<glm_f32x4 *>(out + (size_t)t * d + c) = r;
    if (out_bf16) {
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = f32_to_bf16(r[q]);
      *reinterpret_cast<uint2 *>(out_bf16 + (size_t)t * d + c) =
          uint2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
    }
  }
}

static int hc_slices(int hc, int d) {
  return std::min(kHcMaxSlices, (hc * d + kHcSlice - 1) / kHcSlice);
}

static int check_hc(const char *who, int T, int hc, int d) {
  GLM_REQUIRE(T >= 0 && hc >= 1 && d >= 1, GLM_ERR_INVALID_ARGUMENT, "%s: invalid sizes", who);
  GLM_REQUIRE(hc <= kHcMaxMult, GLM_ERR_UNSUPPORTED_SHAPE, "%s: hc_mult %d > %d", who, hc,
              kHcMaxMult);
  GLM_REQUIRE(d % 4 == 0 && d <= kHcMaxD, GLM_ERR_UNSUPPORTED_SHAPE,
              "%s: hidden size %d must be a multiple of 4 and at most %d", who, d, kHcMaxD);
  return GLM_OK;
}

}  // namespace glm

using namespace glm;

extern "C" size_t glm_hc_workspace_bytes(int T, int hc, int d) {
  if (T < 0 || hc < 1 || hc > kHcMaxMult || d < 1) return 0;
  const size_t M = 2 * hc + hc * hc;
  return (size_t)hc_slices(hc, d) * (size_t)T * (M + 1) * sizeof(float);
}

extern "C" int glm_hc_pre(void *stream, const float *streams, int T, int hc, int d,
                          const float *fn, const float *base, const float *scale,
                          int sinkhorn_iters, float rms_eps, float hc_eps,
                          const float *norm_weight, float norm_eps, int flags, void *workspace,
                          size_t workspace_bytes, float *post, float *comb, float *collapsed,
                          uint16_t *normed) {
  glm::clear_error();
  int rc = check_hc("hc_pre", T, hc, d);
  if (rc) return rc;
  GLM_REQUIRE((flags & ~GLM_HC_BF16_STREAMS) == 0, GLM_ERR_INVALID_ARGUMENT,
              "hc_pre: unknown flags %d", flags);
  GLM_REQUIRE(sinkhorn_iters >= 1, GLM_ERR_INVALID_ARGUMENT, "hc_pre: sinkhorn_iters must be >= 1");
  GLM_REQUIRE(streams && fn && base && scale && post && comb && workspace, GLM_ERR_INVALID_ARGUMENT,
              "hc_pre: null pointer argument");
  GLM_REQUIRE(glm_aligned16({streams, fn, collapsed, workspace}) &&
                  (reinterpret_cast<uintptr_t>(normed) & 7u) == 0,
              GLM_ERR_INVALID_ARGUMENT, "hc_pre: buffers must be 16-byte aligned (normed 8)");
  GLM_REQUIRE(workspace_bytes >= glm_hc_workspace_bytes(T, hc, d), GLM_ERR_WORKSPACE,
              "hc_pre: workspace of %zu bytes, %zu needed", workspace_bytes,
              glm_hc_workspace_bytes(T, hc, d));
  if (T == 0) return GLM_OK;
  const int M = 2 * hc + hc * hc;
  const int S = hc_slices(hc, d);
  float *partial = static_cast<float *>(workspace);
  const dim3 mix_grid(S, (T + kHcTokens - 1) / kHcTokens);
  const int rows = (M + 3) / 4;  // fn rows per wave
  if (rows <= 2)
    hipLaunchKernelGGL(hc_mix_kernel<2>, mix_grid, dim3(kHcThreads), 0, (hipStream_t)stream,
                       streams, fn, T, hc * d, M, partial);
  else if (rows <= 6)
    hipLaunchKernelGGL(hc_mix_kernel<6>, mix_grid, dim3(kHcThreads), 0, (hipStream_t)stream,
                       streams, fn, T, hc * d, M, partial);
  else
    hipLaunchKernelGGL(hc_mix_kernel<20>, mix_grid, dim3(kHcThreads), 0, (hipStream_t)stream,
                       streams, fn, T, hc * d, M, partial);
  GLM_LAUNCH_CHECK("hc_mix_kernel");
  HcFinishArgs a{streams, partial, base, scale, norm_weight, T, hc, d, S, sinkhorn_iters,
                 (flags & GLM_HC_BF16_STREAMS) != 0, rms_eps, hc_eps, norm_eps, post, comb,
                 collapsed, normed};
  hipLaunchKernelGGL(hc_finish_kernel, dim3(T), dim3(kHcThreads), (size_t)d * sizeof(float),
                     (hipStream_t)stream, a);
  GLM_LAUNCH_CHECK("hc_finish_kernel");
  return GLM_OK;
}

// hyper_residual launch for the MoE forward's paths that do not fuse it
int glm_hc_post_launch(hipStream_t stream, const glm::HcFuse &f, const float *y, int T, int d) {
  const int per_block = 4 * kHcThreads;
  const dim3 grid((d + per_block - 1) / per_block, T);
  if (f.bf16)
    hipLaunchKernelGGL(hc_post_kernel<true>, grid, dim3(kHcThreads), 0, stream, f.res, y, f.post,
                       f.comb, f.hc, d, f.out);
  else
    hipLaunchKernelGGL(hc_post_kernel<false>, grid, dim3(kHcThreads), 0, stream, f.res, y, f.post,
                       f.comb, f.hc, d, f.out);
  GLM_LAUNCH_CHECK("hc_post_kernel");
  return GLM_OK;
}

extern "C" int glm_hc_post(void *stream, const float *residual, int T, int hc, int d,
                           const float *y, const float *post, const float *comb, int flags,
                           float *out) {
  glm::clear_error();
  int rc = check_hc("hc_post", T, hc, d);
  if (rc) return rc;
  GLM_REQUIRE((flags & ~GLM_HC_BF16_STREAMS) == 0, GLM_ERR_INVALID_ARGUMENT,
              "hc_post: unknown flags %d", flags);
  GLM_REQUIRE(residual && y && post && comb && out, GLM_ERR_INVALID_ARGUMENT,
              "hc_post: null pointer argument");
  GLM_REQUIRE(glm_aligned16({residual, y, out}), GLM_ERR_INVALID_ARGUMENT,
              "hc_post: buffers must be 16-byte aligned");
  if (T == 0) return GLM_OK;
  const int per_block = 4 * kHcThreads;
  const dim3 grid((d + per_block - 1) / per_block, T);
  if (flags & GLM_HC_BF16_STREAMS)
    hipLaunchKernelGGL(hc_post_kernel<true>, grid, dim3(kHcThreads), 0, (hipStream_t)stream,
                       residual, y, post, comb, hc, d, out);
  else
    hipLaunchKernelGGL(hc_post_kernel<false>, grid, dim3(kHcThreads), 0, (hipStream_t)stream,
                       residual, y, post, comb, hc, d, out);
  GLM_LAUNCH_CHECK("hc_post_kernel");
  return GLM_OK;
}

extern "C" int glm_rms_norm(void *stream, const float *x, int T, int d, const float *weight,
                            float eps, float *out, uint16_t *out_bf16) {
  glm::clear_error();
  GLM_REQUIRE(T >= 0 && d >= 1, GLM_ERR_INVALID_ARGUMENT, "rms_norm: invalid sizes");
  GLM_REQUIRE(d % 4 == 0, GLM_ERR_UNSUPPORTED_SHAPE, "rms_norm: d %% 4 != 0 (d = %d)", d);
  GLM_REQUIRE(x && (out || out_bf16), GLM_ERR_INVALID_ARGUMENT, "rms_norm: null pointer argument");
  GLM_REQUIRE(glm_aligned16({x, out}) && (reinterpret_cast<uintptr_t>(out_bf16) & 7u) == 0,
              GLM_ERR_INVALID_ARGUMENT, "rms_norm: buffers must be 16-byte aligned (bf16 8)");
  if (T == 0) return GLM_OK;
  hipLaunchKernelGGL(rms_norm_kernel, dim3(T), dim3(kHcThreads), 0, (hipStream_t)stream, x, d,
                     weight, eps, out, out_bf16);
  GLM_LAUNCH_CHECK("rms_norm_kernel");
  return GLM_OK;
}
