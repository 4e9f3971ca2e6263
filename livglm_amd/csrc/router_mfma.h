// Router logits for many tokens on f32 MFMA: one workgroup's tile, shared by
// the router's own kernel and the decode path's launch that runs the shared
// expert's gate/up tiles beside it.
#pragma once

#include "glm_common.h"

namespace glm {

// ---------------------------------------------------------------------------
// Logits for many tokens on MFMA: v_mfma_f32_16x16x4_f32 forms exact f32
// products of f32(x) and W and accumulates them in f32 (only the summation
// order differs from a sequential dot product: each wave keeps the even and
// the odd K positions of a step in separate accumulators, added at the end).
// A workgroup's tile (token tile tile_t, expert tile tile_e) = 16 tokens x
// 16 ET experts (ET 16 x 16 tiles: two for many tokens, one for fewer, where
// it doubles a small grid); red holds KSPLIT - 1 partial sums in LDS.  Its
// KSPLIT waves split K into equal ranges
// (4 for many tokens, 16 for fewer, where the grid is small), so several
// waves share each SIMD and hide each other's L2 latency, and the partial
// sums are added in wave order through LDS.  MFMA i of a 32-wide K step takes
// K = k0 + 8q + i in lane (r, q)'s slot, so a lane loads 8 consecutive x
// (16 B of bf16) and 8 consecutive W (32 B) per step.  Rows past T or E are
// clamped for the loads and never stored.
// ---------------------------------------------------------------------------
template <int KSPLIT, int PD, int ET = 2>
__device__ __forceinline__ void router_gemm_tile(const uint16_t *__restrict__ x,
                                                 const float *__restrict__ w, int T, int d, int E,
                                                 float *__restrict__ logits, int tile_t, int tile_e,
                                                 glm_f32x4 (*red)[2][64]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  static_assert(ET == 1 || ET == 2, "one or two expert tiles");
  const int t0 = tile_t * 16;
  const int e0 = tile_e * 16 * ET;
  const int kq = d / KSPLIT;  // this wave's K range [wave * kq, (wave + 1) * kq), a multiple of 32 * PD
  const int kb = wave * kq;
  const uint16_t *xr = x + (size_t)min(t0 + r, T - 1) * d + kb + 8 * q;
  const float *wr0 = w + (size_t)min(e0 + r, E - 1) * d + kb + 8 * q;
  const float *wr1 = w + (size_t)min(e0 + 16 + r, E - 1) * d + kb + 8 * q;
  glm_f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  glm_f32x4 acc2 = {0.f, 0.f, 0.f, 0.f}, acc3 = {0.f, 0.f, 0.f, 0.f};
  // a ring of PD steps of operands in registers: step s + PD is in flight
  // while step s feeds the MFMAs (L2 latency spans many steps' MFMAs)
  glm_u32x4 xv[PD];
  float4 wa0[PD], wb0[PD], wa1[PD], wb1[PD];
#pragma unroll
  for (int i = 0; i < PD; ++i) {
    xv[i] = *reinterpret_cast<const glm_u32x4 *>(xr + 32 * i);
    wa0[i] = *reinterpret_cast<const float4 *>(wr0 + 32 * i);
    wb0[i] = *reinterpret_cast<const float4 *>(wr0 + 32 * i + 4);
    wa1[i] = *reinterpret_cast<const float4 *>(wr1 + 32 * i);
    wb1[i] = *reinterpret_cast<const float4 *>(wr1 + 32 * i + 4);
  }
  for (int k0 = 0; k0 < kq; k0 += 32 * PD) {
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      const glm_u32x4 cx = xv[i];
      const float4 ca0 = wa0[i], cb0 = wb0[i], ca1 = wa1[i], cb1 = wb1[i];
      const int kn = k0 + 32 * (i + PD);
      if (kn < kq) {
        xv[i] = *reinterpret_cast<const glm_u32x4 *>(xr + kn);
        wa0[i] = *reinterpret_cast<const float4 *>(wr0 + kn);
        wb0[i] = *reinterpret_cast<const float4 *>(wr0 + kn + 4);
        wa1[i] = *reinterpret_cast<const float4 *>(wr1 + kn);
        wb1[i] = *reinterpret_cast<const float4 *>(wr1 + kn + 4);
      }
      const float xf[8] = {bf16_to_f32(cx[0] & 0xffffu), bf16_to_f32(cx[0] >> 16),
                           bf16_to_f32(cx[1] & 0xffffu), bf16_to_f32(cx[1] >> 16),
                           bf16_to_f32(cx[2] & 0xffffu), bf16_to_f32(cx[2] >> 16),
                           bf16_to_f32(cx[3] & 0xffffu), bf16_to_f32(cx[3] >> 16)};
      const float w0[8] = {ca0.x, ca0.y, ca0.z, ca0.w, cb0.x, cb0.y, cb0.z, cb0.w};
      const float w1[8] = {ca1.x, ca1.y, ca1.z, ca1.w, cb1.x, cb1.y, cb1.z, cb1.w};
      // four independent accumulation chains keep the MFMA pipeline full
#pragma unroll
      for (int m = 0; m < 8; m += 2) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[m], w0[m], acc0, 0, 0, 0);
        if constexpr (ET == 2)
          acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[m], w1[m], acc1, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[m + 1], w0[m + 1], acc2, 0, 0, 0);
        if constexpr (ET == 2)
          acc3 = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[m + 1], w1[m + 1], acc3, 0, 0, 0);
      }
    }
  }
  acc0 += acc2;
  acc1 += acc3;
  if (wave > 0) {
    red[wave - 1][0][lane] = acc0;
    red[wave - 1][1][lane] = acc1;
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int j = 0; j < KSPLIT - 1; ++j) {
    acc0 += red[j][0][lane];
    acc1 += red[j][1][lane];
  }
  // lane (r, q) holds tokens 4q..4q+3 of the 16 for experts e0 + r, e0 + 16 + r
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int t = t0 + 4 * q + m;
    if (t >= T) continue;
    if (e0 + r < E) logits[(size_t)t * E + e0 + r] = acc0[m];
    if (ET == 2 && e0 + 16 + r < E) logits[(size_t)t * E + e0 + 16 + r] = acc1[m];
  }
}

}  // namespace glm
