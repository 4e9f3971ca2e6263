// Router: logits GEMV + sigmoid/bias/group-mask/top-k/normalise.
// Restates TopKRouter.__call__ (moe.py:36-63) for gfx950.
#include "glm_common.h"
#include "lds_stage.h"
#include "router_mfma.h"
#include "topk_select.h"

namespace glm {

// ---------------------------------------------------------------------------
// logits[t][e] = sum_i f32(x[t][i]) * w[e][i]
//
// One wave owns one expert row of W (read once per TT-token pass, 16 B per
// lane per step, fully coalesced) and TT tokens; lane l accumulates the K
// positions 4l + 256s.  The final f32 value is a butterfly wave sum.
// ---------------------------------------------------------------------------
template <int TT>
__global__ __launch_bounds__(256) void router_logits_kernel(const uint16_t *__restrict__ x,
                                                            const float *__restrict__ w, int T,
                                                            int d, int E,
                                                            float *__restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int t0 = blockIdx.y * TT;
  if (e >= E) return;
  const float *wrow = w + (size_t)e * d;
  float acc[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = 0.0f;
  const int nt = min(TT, T - t0);
  for (int k = lane * 4; k < d; k += 256) {
    const float4 wv = *reinterpret_cast<const float4 *>(wrow + k);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t < nt) {
        const uint2 xv = *reinterpret_cast<const uint2 *>(x + (size_t)(t0 + t) * d + k);
        float a = acc[t];
        a = fmaf(bf16_to_f32(xv.x & 0xffffu), wv.x, a);
        a = fmaf(bf16_to_f32(xv.x >> 16), wv.y, a);
        a = fmaf(bf16_to_f32(xv.y & 0xffffu), wv.z, a);
        a = fmaf(bf16_to_f32(xv.y >> 16), wv.w, a);
        acc[t] = a;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    if (t < nt) {
      const float v = wave_sum(acc[t]);
      if (lane == 0) logits[(size_t)(t0 + t) * E + e] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Logits for many tokens on f32 MFMA (router_gemm_tile): grid (token tiles,
// expert tiles).
// ---------------------------------------------------------------------------
template <int KSPLIT, int PD, int ET = 2>
__global__ __launch_bounds__(64 * KSPLIT) void router_gemm_kernel(
    const uint16_t *__restrict__ x, const float *__restrict__ w, int T, int d, int E,
    float *__restrict__ logits) {
  __shared__ glm_f32x4 red[KSPLIT - 1][2][64];
  router_gemm_tile<KSPLIT, PD, ET>(x, w, T, d, E, logits, blockIdx.x, blockIdx.y, red);
}

// ---------------------------------------------------------------------------
// Logits for many tokens on bf16 MFMA.  The f32 router weights are first split
// into three bf16 parts, w = w0 + w1 + w2 (w0 = bf16(w), w1 = bf16(w - w0),
// w2 = bf16(w - w0 - w1); the f32 significand's 24 bits fit three bf16
// significands, exactly for 2^-100 <= |w| < 2^127 and to within 2^-133 below),
// so x . w = x . w0 + x . w1 + x . w2 with every product exact (bf16 x bf16)
// and f32 accumulation: the f32 dot product up to the summation order, at the
// bf16 MFMA rate (a 32-wide K step is three bf16 MFMAs per tile instead of
// eight f32 ones).
// Workgroup = 64 tokens x 32 experts, eight waves, one 16 x 16 output tile
// each over the whole of K.  K advances in chunks of 128: the chunk's 64 token
// rows and 96 split-weight rows (3 parts x 32 experts) are staged in LDS by
// direct-to-LDS wave loads of 4 rows x 256 B (whole cache lines), three stages
// deep; piece p (16 bytes) of staged row R sits at p ^ (R & 15), so the MFMA
// operand reads (16 rows x one piece column) spread over the banks.  (Chunks
// of 64 ran a workgroup barrier per 6 MFMAs of a wave: 16.3 us at T = 4096,
// E = 128, d = 2048.  Loads of 16 rows x 64 B straight into registers, one
// MFMA operand per lane, ran at ~28 GB/s per CU: 23.2 us.)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void router_weight_split_kernel(const float *__restrict__ w,
                                                                  long long n,
                                                                  uint16_t *__restrict__ ws) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) bf16x3_split_one(w, n, ws, i);
}

constexpr int kSplitRouterWaves = 8;
constexpr int kRouterChunk = 128;               // K per stage
constexpr int kRouterRowBytes = kRouterChunk * 2;
constexpr int kRouterRows = 64 + 96;            // staged rows per chunk: tokens, then 3 x 32 weights
constexpr int kRouterStageBytes = kRouterRows * kRouterRowBytes;
constexpr int kRouterStages = 3;
constexpr int kRouterRowsPerLoad = 1024 / kRouterRowBytes;            // 4
constexpr int kRouterWaveLoads = kRouterRows / kRouterRowsPerLoad;    // 40 wave loads of 1 KB
constexpr int kRouterLoads = kRouterWaveLoads / kSplitRouterWaves;    // 5 per wave
static_assert(kRouterLoads * kSplitRouterWaves == kRouterWaveLoads, "loads split evenly");
static_assert(64 % kRouterRowsPerLoad == 0, "a load stages token rows or weight rows");
static_assert(kRouterStages == 3, "the ring's wait counts");
static_assert(kRouterStages * kRouterStageBytes <= 160 * 1024, "LDS ring exceeds 160 KB");

__global__ __launch_bounds__(64 * kSplitRouterWaves) void router_gemm_bf16x3_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ ws, int T, int d, int E,
    float *__restrict__ logits) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // kRouterStages stages
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int t0 = blockIdx.x * 64;
  const int e0 = blockIdx.y * 32;
  const int nchunks = d / kRouterChunk;
  // load j of wave w stages rows 4 g .. 4 g + 3, g = 8 j + w; lane l fetches
  // piece (l & 15) ^ (row & 15) of row 4 g + (l >> 4)
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, (uint32_t)((size_t)T * d * 2));
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(ws, (uint32_t)((size_t)3 * E * d * 2));
  uint32_t voff[kRouterLoads];
#pragma unroll
  for (int j = 0; j < kRouterLoads; ++j) {
    const int g = kSplitRouterWaves * j + wave;
    const int row = kRouterRowsPerLoad * g + (lane >> 4), piece = (lane & 15) ^ (row & 15);
    size_t src_row;
    if (row < 64) {
      src_row = (size_t)min(t0 + row, T - 1);
    } else {
      const int wr = row - 64, part = wr / 32;
      src_row = (size_t)part * E + min(e0 + wr % 32, E - 1);
    }
    voff[j] = (uint32_t)(src_row * d * 2) + 16u * piece;
  }
  auto issue = [&](int c, int stage) {
    uint8_t *base = smem + stage * kRouterStageBytes;
#pragma unroll
    for (int j = 0; j < kRouterLoads; ++j) {
      const int g = kSplitRouterWaves * j + wave;  // token rows: g < 16
      buf16_to_lds(g < 64 / kRouterRowsPerLoad ? xrs : wrs, base + g * 1024, voff[j],
                   c * kRouterRowBytes);
    }
  };
  // this wave's output tile: tokens 16 tt .. + 15, experts 16 et .. + 15
  const int tt = wave >> 1, et = wave & 1;
  glm_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int stage) {
    const uint8_t *base = smem + stage * kRouterStageBytes;
#pragma unroll
    for (int i = 0; i < kRouterChunk / 32; ++i) {
      const int xr = 16 * tt + r;
      const glm_bf16x8 xa = *reinterpret_cast<const glm_bf16x8 *>(
          base + xr * kRouterRowBytes + 16 * ((4 * i + q) ^ (xr & 15)));
      glm_bf16x8 wb[3];
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        const int wr = 64 + 32 * p + 16 * et + r;
        wb[p] = *reinterpret_cast<const glm_bf16x8 *>(base + wr * kRouterRowBytes +
                                                      16 * ((4 * i + q) ^ (wr & 15)));
      }
#pragma unroll
      for (int p = 0; p < 3; ++p)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, wb[p], acc, 0, 0, 0);
    }
  };
  // ring: chunks c + 1 and c + 2 in flight while c is consumed; the barrier
  // of iteration c also guarantees that every wave is done with chunk c - 1,
  // whose stage the loads of chunk c + 2 overwrite
  issue(0, 0);
  if (nchunks > 1) issue(1, 1);
  for (int c = 0; c < nchunks; ++c) {
    if (c + 1 < nchunks)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRouterLoads));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    ring_barrier();
    if (c + 2 < nchunks) issue(c + 2, (c + 2) % kRouterStages);
    compute(c % kRouterStages);
  }
  // lane (r, q) holds tokens 4q..4q+3 of the tile for expert e0 + 16 et + r
  const int e = e0 + 16 * et + r;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int t = t0 + 16 * tt + 4 * q + m;
    if (t < T && e < E) logits[(size_t)t * E + e] = acc[m];
  }
}

// ---------------------------------------------------------------------------
// Selection: one wave per token (select_token), four tokens per workgroup.
// ---------------------------------------------------------------------------
template <int EPL>
__global__ __launch_bounds__(256) void router_select_kernel(
    const float *__restrict__ logits, const float *__restrict__ bias, int T, int E, int k,
    int n_group, int topk_group, int norm, float scale, float *__restrict__ weights,
    uint32_t *__restrict__ indices) {
  __shared__ float scratch[4][64 * EPL + 256];
  __shared__ int sel[4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;  // wave-uniform; the selection synchronises one wave only
  select_token<EPL>(logits + (size_t)t * E, bias, E, k, n_group, topk_group, norm, scale,
                    weights + (size_t)t * k, indices + (size_t)t * k, sel[wave], scratch[wave],
                    lane);
}


}  // namespace glm

// Launches the router; `logits` must be a valid [T][E] buffer here.
// Router logits only (no selection): the MFMA kernel for 16 or more tokens.
bool glm_router_gemm_supported(int T, int d) {
  return (T >= 256 && d % (32 * 4) == 0) || (T >= 16 && d % (32 * 16) == 0);
}

int glm_router_logits_launch(hipStream_t stream, const uint16_t *x, int T, int d,
                             const float *weight, int E, float *logits) {
  using namespace glm;
  if (!glm_router_gemm_supported(T, d)) {
    glm::set_error("router logits: unsupported T=%d d=%d", T, d);
    return GLM_ERR_UNSUPPORTED_SHAPE;
  }
  // template arguments: K split (waves), 32-wide K steps in flight per wave,
  // 16-expert tiles per workgroup
  dim3 grid((T + 15) / 16, (E + 31) / 32);
  if (T < 256 && d % (32 * 16 * 2) == 0) {
    // fewer than 256 tokens: one 16-expert tile per workgroup, twice the grid
    grid.y = (E + 15) / 16;
    hipLaunchKernelGGL((router_gemm_kernel<16, 2, 1>), grid, dim3(1024), 0, stream, x, weight, T, d, E, logits);
  } else if (T >= 256 && d % (32 * 4) == 0) {
    if (d % (32 * 4 * 4) == 0)
      hipLaunchKernelGGL((router_gemm_kernel<4, 4>), grid, dim3(256), 0, stream, x, weight, T, d, E, logits);
    else
      hipLaunchKernelGGL((router_gemm_kernel<4, 1>), grid, dim3(256), 0, stream, x, weight, T, d, E, logits);
  } else {
    if (d % (32 * 16 * 2) == 0)  // 1024-thread blocks: at most 128 registers, so two steps
      hipLaunchKernelGGL((router_gemm_kernel<16, 2>), grid, dim3(1024), 0, stream, x, weight, T, d, E, logits);
    else
      hipLaunchKernelGGL((router_gemm_kernel<16, 1>), grid, dim3(1024), 0, stream, x, weight, T, d, E, logits);
  }
  GLM_LAUNCH_CHECK("router_gemm_kernel");
  return GLM_OK;
}

// Top-k selection of precomputed logits, one wave per token.
int glm_router_select_launch(hipStream_t stream, const float *logits, const float *bias, int T,
                             int E, int k, int n_group, int topk_group, int norm, float scale,
                             float *weights, uint32_t *indices) {
  using namespace glm;
  if (T == 0) return GLM_OK;
  const int epl = (E + 63) / 64;
#define GLM_SELECT(N)                                                                         \
  hipLaunchKernelGGL(router_select_kernel<N>, dim3((T + 3) / 4), dim3(256), 0, stream, logits, bias, T, \
                     E, k, n_group, topk_group, norm, scale, weights, indices)
  if (epl <= 1) GLM_SELECT(1);
  else if (epl <= 2) GLM_SELECT(2);
  else if (epl <= 4) GLM_SELECT(4);
  else if (epl <= 8) GLM_SELECT(8);
  else GLM_SELECT(16);
#undef GLM_SELECT
  GLM_LAUNCH_CHECK("router_select_kernel");
  return GLM_OK;
}

// Whether the bf16-split router GEMM covers this call (it needs
// glm_router_split_bytes of scratch for the split weights).
bool glm_router_split_supported(int T, int d) {
  // (the staged loads address x through a 32-bit buffer range)
  return T >= 256 && d % (64 * glm::kSplitRouterWaves) == 0 && (size_t)T * d * 2 < (1ull << 32);
}

size_t glm_router_split_bytes(int E, int d) { return (size_t)3 * E * d * 2; }

int glm_router_launch(hipStream_t stream, const uint16_t *x, int T, int d, const float *weight,
                      const float *bias, int E, int k, int n_group, int topk_group, int norm,
                      float scale, float *logits, float *weights, uint32_t *indices,
                      uint16_t *wsplit, bool wsplit_ready) {
  using namespace glm;
  if (T == 0) return GLM_OK;
  if (wsplit != nullptr && glm_router_split_supported(T, d)) {
    const long long n = (long long)E * d;
    if (!wsplit_ready) {
      hipLaunchKernelGGL(router_weight_split_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                         0, stream, weight, n, wsplit);
      GLM_LAUNCH_CHECK("router_weight_split_kernel");
    }
    const dim3 grid((T + 63) / 64, (E + 31) / 32);
    hipLaunchKernelGGL(router_gemm_bf16x3_kernel, grid, dim3(64 * kSplitRouterWaves),
                       (size_t)kRouterStages * kRouterStageBytes, stream, x,
                       wsplit, T, d, E, logits);
  } else if (glm_router_gemm_supported(T, d)) {
    const int rc = glm_router_logits_launch(stream, x, T, d, weight, E, logits);
    if (rc) return rc;
  } else if (T <= 2) {
    dim3 grid((E + 3) / 4, (T + 1) / 2);
    hipLaunchKernelGGL(router_logits_kernel<2>, grid, dim3(256), 0, stream, x, weight, T, d, E,
                       logits);
  } else {
    dim3 grid((E + 3) / 4, (T + 7) / 8);
    hipLaunchKernelGGL(router_logits_kernel<8>, grid, dim3(256), 0, stream, x, weight, T, d, E,
                       logits);
  }
  GLM_LAUNCH_CHECK("router_logits_kernel");
  return glm_router_select_launch(stream, logits, bias, T, E, k, n_group, topk_group, norm, scale,
                                  weights, indices);
}

int glm_router_validate(const void *x, int T, int d, const void *weight, const void *bias, int E,
                        int k, int n_group, int topk_group, const void *weights,
                        const void *indices) {
  GLM_REQUIRE(x && weight && bias && weights && indices, GLM_ERR_INVALID_ARGUMENT,
              "router: null pointer argument");
  GLM_REQUIRE(T >= 0 && d > 0 && E > 0, GLM_ERR_INVALID_ARGUMENT,
              "router: invalid sizes T=%d d=%d E=%d", T, d, E);
  GLM_REQUIRE(d % 4 == 0, GLM_ERR_UNSUPPORTED_SHAPE, "router: d=%d must be a multiple of 4", d);
  GLM_REQUIRE(E <= 1024, GLM_ERR_UNSUPPORTED_SHAPE, "router: E=%d exceeds 1024", E);
  GLM_REQUIRE(k >= 1 && k <= E, GLM_ERR_INVALID_ARGUMENT, "router: invalid top-k %d for E=%d",
              k, E);
  GLM_REQUIRE(k <= 64, GLM_ERR_UNSUPPORTED_SHAPE, "router: top-k %d exceeds 64", k);
  GLM_REQUIRE(glm_aligned16({x, weight, bias, weights, indices}), GLM_ERR_INVALID_ARGUMENT,
              "router: buffers must be 16-byte aligned");
  GLM_REQUIRE(n_group >= 1 && n_group <= 64 && E % n_group == 0 && E / n_group >= 2,
              GLM_ERR_INVALID_ARGUMENT, "router: invalid n_group=%d for E=%d", n_group, E);
  GLM_REQUIRE(topk_group >= 1 && topk_group <= n_group, GLM_ERR_INVALID_ARGUMENT,
              "router: invalid topk_group=%d", topk_group);
  return GLM_OK;
}

extern "C" int glm_router_topk(void *stream, const uint16_t *x, int T, int d, const float *weight,
                               const float *bias, int E, int top_k, int n_group, int topk_group,
                               int norm_topk_prob, float routed_scaling_factor, float *logits,
                               float *weights, uint32_t *indices) {
  glm::clear_error();
  int rc = glm_router_validate(x, T, d, weight, bias, E, top_k, n_group, topk_group, weights,
                               indices);
  if (rc != GLM_OK) return rc;
  GLM_REQUIRE(logits != nullptr, GLM_ERR_INVALID_ARGUMENT,
              "router: logits buffer is required by this entry point");
  return glm_router_launch((hipStream_t)stream, x, T, d, weight, bias, E, top_k, n_group,
                           topk_group, norm_topk_prob, routed_scaling_factor, logits, weights,
                           indices, nullptr, false);
}
