// Decode-size routed-MoE layer (T <= 64, T*k <= 512 pairs) in five kernels:
//
//   1. route_logits_kernel    router logits (one block per expert, 4 waves
//                             split d) -- and, in extra blocks, the bf16
//                             shared expert's gate/up tiles, which do not
//                             depend on routing and so overlap with it.
//   2. select_dispatch_kernel block 0: top-k selection of every token
//                             (moe.py:39-62) and the dispatch -- histogram,
//                             exclusive scan, stable permute, work list -- in
//                             LDS; extra blocks: the shared expert's down tiles.
//   3. decode_gate_up_kernel  routed MXFP4 gate/up + SwiGLU, one group of
//                             tiles per active expert slot.
//   4. decode_down_kernel     routed MXFP4 down.
//   5. combine_kernel         weighted top-k merge + shared add.
//
// With very few tokens (T <= 4, k <= 8) experts are rarely shared between
// tokens, so the layer runs token-major in three kernels and skips the
// dispatch altogether:
//
//   1. route_logits_kernel    as above.
//   2. select_gate_up_kernel  block = (pair t*k + j, 16-row tile): every wave
//                             selects token t's experts from its logits, then
//                             the block computes gate/up + SwiGLU of expert j
//                             for that token; extra blocks: shared down tiles.
//   3. down_combine_kernel    block = (token, 16 rows of d): wave j runs the
//                             down projection of the token's expert j, and the
//                             weighted merge + shared add happen in LDS in the
//                             combine's order.
//
// Every kernel boundary is a stream-ordered dependency; nothing synchronises
// across blocks inside a kernel, and every reduction runs in one fixed order.
#include "mfma_tile.h"
#include "scalex_tile.h"
#include "router_mfma.h"
#include "topk_select.h"

int glm_router_select_launch(hipStream_t stream, const float *logits, const float *bias, int T,
                             int E, int k, int n_group, int topk_group, int norm, float scale,
                             float *weights, uint32_t *indices);
int glm_router_logits_launch(hipStream_t stream, const uint16_t *x, int T, int d,
                             const float *weight, int E, float *logits);
bool glm_router_gemm_supported(int T, int d);

namespace glm {

constexpr int kRouteThreads = 256;
constexpr int kMaxFusedPairs = 512;  // T*k handled by the fused route kernel
constexpr int kFusedMaxE = 448;

struct RouteArgs {
  const uint16_t *x;
  const float *w;
  const float *bias;
  int T, d, E, k, n_group, topk_group, norm;
  float scale;
  float *logits;
  float *weights;
  uint32_t *indices;
  int32_t *counts, *offsets, *perm, *inv, *pair_token, *active, *num_active, *status;
  int4 *work;
  int presel;  // select_dispatch_kernel: indices already selected (router_select_kernel)
  int logits_done;  // route_logits_kernel: logits already computed; run the shared blocks only
};

// Exclusive scan over a 256-thread block (4 waves); *total gets the sum.
__device__ __forceinline__ int scan256(int v, int *s_tmp, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) s_tmp[wave] = incl;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int s = s_tmp[w];
    if (w < wave) base += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + incl - v;
}

// The bf16 shared expert (DenseMLP, layers.py:160-171) as tiles that ride in
// the routing kernels.  Gate/up tiles are 16 rows; with few tokens (skq > 1)
// their K range is split over skq tiles that write f32 partial sums, which the
// down tiles add in order and turn into bf16 SwiGLU activations in LDS;
// otherwise gate/up tiles cover all of d and write bf16 activations.  Down
// tiles are 64 rows x Is/skd and write f32 partial sums [skd][T][d] that the
// combine adds in order (all partial sums are exact f32 reductions of
// disjoint K ranges, so the result is the f32 dot product rounded once).
constexpr int kMaxSkq = 8;  // gate/up K ranges of the few-token shared tiles (d <= 4096)

struct SharedArgs {
  const uint16_t *x;
  const uint8_t *sg, *su, *sd;  // bf16 gate/up [Is][d], down [d][Is] (sg == nullptr: none)
  int T, d, Is, skq, skd, gu_blocks, dn_blocks;
  float *gp, *up;  // skq > 1: gate/up partial sums [skq][T][Is]
  uint16_t *hs;    // skq == 1: activations [T][Is]
  float *yp;       // down partial sums [skd][T][d]
  float limit;
};

template <int CPW>
__device__ void shared_gate_up_tile(const SharedArgs &a, int b, glm_f32x4 *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int d = a.d;
  const uint8_t *srow[2] = {nullptr, nullptr};
  if (a.skq > 1) {
    const int row0 = (b / a.skq) * 16;
    const int kq = b % a.skq;
    const int kbase = kq * (d / a.skq) + wave * 128;
    const uint8_t *wrow[2] = {a.sg + (size_t)(row0 + r) * d * 2, a.su + (size_t)(row0 + r) * d * 2};
    for (int p0 = 0; p0 < a.T; p0 += 16) {
      const int t = p0 + r;
      const uint16_t *act = a.x + (size_t)min(t, a.T - 1) * d;  // padding: any valid row
      glm_f32x4 acc[2] = {glm_f32x4{0.f, 0.f, 0.f, 0.f}, glm_f32x4{0.f, 0.f, 0.f, 0.f}};
      wave_mma<FMT_BF16, 2, 1, false>(wrow, srow, kbase, q, act, acc);
      if (ksplit_reduce<2>(acc, red, wave, 4, lane) && t < a.T) {
        const size_t o = ((size_t)kq * a.T + t) * a.Is + row0 + 4 * q;
        *reinterpret_cast<glm_f32x4 *>(a.gp + o) = acc[0];
        *reinterpret_cast<glm_f32x4 *>(a.up + o) = acc[1];
      }
    }
  } else {
    // full-K tiles, one block per (16-row tile, group of 16 tokens)
    const int tiles = a.Is / 16;
    const int row0 = (b % tiles) * 16;
    const int kbase = wave * CPW * 128;
    const uint8_t *wrow[2] = {a.sg + (size_t)(row0 + r) * d * 2, a.su + (size_t)(row0 + r) * d * 2};
    for (int p0 = (b / tiles) * 16; p0 < min(a.T, (b / tiles) * 16 + 16); p0 += 16) {
      const int t = p0 + r;
      const uint16_t *act = a.x + (size_t)min(t, a.T - 1) * d;  // padding: any valid row
      glm_f32x4 acc[2] = {glm_f32x4{0.f, 0.f, 0.f, 0.f}, glm_f32x4{0.f, 0.f, 0.f, 0.f}};
      wave_mma<FMT_BF16, 2, CPW>(wrow, srow, kbase, q, act, acc);
      if (ksplit_reduce<2>(acc, red, wave, 4, lane) && t < a.T) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
          o[m] = f32_to_bf16(limited_swiglu(bf16_round(acc[0][m]), bf16_round(acc[1][m]), a.limit));
        store_rows4(a.hs + (size_t)t * a.Is + row0 + 4 * q, o);
      }
    }
  }
}

// The same full-K tile (16 rows, one group of 16 tokens) computed by 16 waves
// that split K, CPW 128-wide chunks each: the workgroups that run beside the
// router's tiles in router_shared_kernel, where a wave's whole K range goes
// out in one round trip.
constexpr int kRouterShWaves = 16;

template <int CPW>
__device__ void shared_gate_up_tile16(const SharedArgs &a, int b, glm_f32x4 *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int d = a.d;
  const int tiles = a.Is / 16;
  const int row0 = (b % tiles) * 16;
  const int t = (b / tiles) * 16 + r;
  const int kbase = wave * CPW * 128;
  const uint8_t *wrow[2] = {a.sg + (size_t)(row0 + r) * d * 2, a.su + (size_t)(row0 + r) * d * 2};
  const uint8_t *srow[2] = {nullptr, nullptr};
  const uint16_t *act = a.x + (size_t)min(t, a.T - 1) * d;  // padding: any valid row
  glm_f32x4 acc[2] = {glm_f32x4{0.f, 0.f, 0.f, 0.f}, glm_f32x4{0.f, 0.f, 0.f, 0.f}};
  wave_mma<FMT_BF16, 2, CPW>(wrow, srow, kbase, q, act, acc);
  if (ksplit_reduce<2>(acc, red, wave, kRouterShWaves, lane) && t < a.T) {
    uint32_t o[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
      o[m] = f32_to_bf16(limited_swiglu(bf16_round(acc[0][m]), bf16_round(acc[1][m]), a.limit));
    store_rows4(a.hs + (size_t)t * a.Is + row0 + 4 * q, o);
  }
}

// Router logits on f32 MFMA (router_gemm_tile, 16-expert tiles, blocks
// [0, router_blocks), token tile fastest) with the shared expert's full-K
// gate/up tiles as the workgroups after them: both need only x, and the
// router's small grid leaves most CUs free.
template <int CPW>
__global__ __launch_bounds__(64 * kRouterShWaves) void router_shared_kernel(
    const uint16_t *x, const float *w, int T, int d, int E, float *logits, int token_tiles,
    int router_blocks, SharedArgs sh) {
  __shared__ glm_f32x4 red[kRouterShWaves - 1][2][64];
  const int b = blockIdx.x;
  if (b < router_blocks) {
    router_gemm_tile<kRouterShWaves, 2, 1>(x, w, T, d, E, logits, b % token_tiles,
                                           b / token_tiles, red);
    return;
  }
  shared_gate_up_tile16<CPW>(sh, b - router_blocks, &red[0][0][0]);
}

template <int CPW_S>
__device__ void shared_down_tile(const SharedArgs &a, int b, uint16_t *s_h) {
  constexpr int KS = CPW_S * 128;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int d = a.d;
  // with full-K gate/up tiles (skq == 1) the blocks also split the tokens
  // into groups of 16
  const int per_group = (d / 64) * a.skd;
  const int tgroup = a.skq > 1 ? 0 : b / per_group;
  b = a.skq > 1 ? b : b % per_group;
  const int tile = b / a.skd, kd = b % a.skd;
  const int row0 = tile * 64 + wave * 16;
  const int kbase = kd * KS;
  if (a.skq > 1) {
    // few tokens (one group of 16): the tile's weights go out first -- they
    // depend on nothing -- then the gate/up partial sums, two elements per
    // thread at a time with every K range's load in flight together (ranges
    // past skq re-read the last and are not added)
    const uint8_t *wp = a.sd + ((size_t)(row0 + r) * a.Is + kbase) * 2;
    WChunk<FMT_BF16> w[CPW_S];
#pragma unroll
    for (int c = 0; c < CPW_S; ++c) w[c] = load_bf16_chunk<false>(wp, c * 128, q);
    for (int i0 = 0; i0 < a.T * KS; i0 += 512) {
      float gv[2][kMaxSkq], uv[2][kMaxSkq];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = min(i0 + (int)threadIdx.x + 256 * u, a.T * KS - 1);
        const int t = i / KS, kk = kbase + i % KS;
#pragma unroll
        for (int qq = 0; qq < kMaxSkq; ++qq) {
          const size_t o = ((size_t)min(qq, a.skq - 1) * a.T + t) * a.Is + kk;
          gv[u][qq] = a.gp[o];
          uv[u][qq] = a.up[o];
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = i0 + (int)threadIdx.x + 256 * u;
        float g = gv[u][0], up = uv[u][0];
#pragma unroll
        for (int qq = 1; qq < kMaxSkq; ++qq) {
          if (qq < a.skq) {
            g += gv[u][qq];
            up += uv[u][qq];
          }
        }
        if (i < a.T * KS)
          s_h[i] = (uint16_t)f32_to_bf16(limited_swiglu(bf16_round(g), bf16_round(up), a.limit));
      }
    }
    __syncthreads();
    const int t = r;
    const uint16_t *act = s_h + (size_t)min(t, a.T - 1) * KS;  // padding columns read a valid row
    glm_f32x4 acc = glm_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CPW_S; ++c) {
      glm_bf16x8 wa[4], xb[4];
      chunk_frags<FMT_BF16>(w[c], 0u, wa);
      load_act_frags(act, c * 128, q, xb);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[i], xb[i], acc, 0, 0, 0);
    }
    if (t < a.T)
      *reinterpret_cast<glm_f32x4 *>(a.yp + ((size_t)kd * a.T + t) * d + row0 + 4 * q) = acc;
    return;
  }
  const uint8_t *wrow[1] = {a.sd + ((size_t)(row0 + r) * a.Is + kbase) * 2};
  const uint8_t *srow[1] = {nullptr};
  for (int p0 = tgroup * 16; p0 < min(a.T, tgroup * 16 + 16); p0 += 16) {
    const int t = p0 + r;
    glm_f32x4 acc[1] = {glm_f32x4{0.f, 0.f, 0.f, 0.f}};
    const int tc = min(t, a.T - 1);  // padding columns read a valid row
    const uint16_t *act = a.hs + (size_t)tc * a.Is + kbase;
    wave_mma<FMT_BF16, 1, CPW_S>(wrow, srow, 0, q, act, acc);
    if (t < a.T)
      *reinterpret_cast<glm_f32x4 *>(a.yp + ((size_t)kd * a.T + t) * d + row0 + 4 * q) = acc[0];
  }
}

// logits[t][e] = f32(x[t]) . w[e] for all tokens; block = expert e, wave w
// sums the K range [w*d/4, (w+1)*d/4), partials added in wave order.
template <int TT, int CPW>
__global__ __launch_bounds__(kRouteThreads) void route_logits_kernel(RouteArgs a, SharedArgs sh) {
  __shared__ float s_part[4][TT];
  __shared__ glm_f32x4 red[3 * 2 * 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x + (a.logits_done ? a.E : 0);
  const int T = a.T, d = a.d, E = a.E;
  if (e >= E) {
    shared_gate_up_tile<CPW>(sh, e - E, red);
    return;
  }
  const int kq = d >> 2;
  const float *wrow = a.w + (size_t)e * d + wave * kq;
  auto fma4 = [](float &acc, float4 wv, uint2 xv) {
    float s = acc;
    s = fmaf(bf16_to_f32(xv.x & 0xffffu), wv.x, s);
    s = fmaf(bf16_to_f32(xv.x >> 16), wv.y, s);
    s = fmaf(bf16_to_f32(xv.y & 0xffffu), wv.z, s);
    s = fmaf(bf16_to_f32(xv.y >> 16), wv.w, s);
    acc = s;
  };
  for (int t0 = 0; t0 < T; t0 += TT) {
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = 0.0f;
    // tokens past T re-read the last row (never stored): branch-free
    // loads are all in flight at once
    int kk0 = lane * 4;
    if constexpr (TT <= 2) {
      // the row's first four rounds of 256 (all of K up to d = 4096) are
      // loaded together, so it arrives in one memory round trip; the sums
      // still run in K order
      constexpr int kRounds = 4;
      float4 wv[kRounds];
#pragma unroll
      for (int u = 0; u < kRounds; ++u)
        if (kk0 + 256 * u < kq) wv[u] = *reinterpret_cast<const float4 *>(wrow + kk0 + 256 * u);
#pragma unroll
      for (int u = 0; u < kRounds; ++u) {
        const int kk = kk0 + 256 * u;
        if (kk < kq) {
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            const int tt = min(t0 + t, T - 1);
            fma4(acc[t], wv[u], *reinterpret_cast<const uint2 *>(a.x + (size_t)tt * d + wave * kq + kk));
          }
        }
      }
      kk0 += 256 * kRounds;
    }
    for (int kk = kk0; kk < kq; kk += 256) {
      const float4 wv = *reinterpret_cast<const float4 *>(wrow + kk);
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int tt = min(t0 + t, T - 1);
        fma4(acc[t], wv, *reinterpret_cast<const uint2 *>(a.x + (size_t)tt * d + wave * kq + kk));
      }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const float v = wave_sum(acc[t]);
      if (lane == 0) s_part[wave][t] = v;
    }
    __syncthreads();
    if (threadIdx.x < TT && t0 + (int)threadIdx.x < T) {
      const int t = threadIdx.x;
      a.logits[(size_t)(t0 + t) * E + e] = ((s_part[0][t] + s_part[1][t]) + s_part[2][t]) + s_part[3][t];
    }
    __syncthreads();
  }
}

// Logits already on the MFMA router: the per-token selection (one wave per
// token, four tokens per block: blocks [0, sel)) rides beside the shared
// expert's gate/up tiles (the blocks after them), which need only x.
template <int CPW, int EPL>
__global__ __launch_bounds__(kRouteThreads) void select_shared_kernel(RouteArgs a, SharedArgs sh) {
  constexpr int kSelWords = 4 * (64 * EPL + 256) + 4 * 64;
  constexpr int kRedWords = 3 * 2 * 64 * 4;
  __shared__ __align__(16) float lds[kSelWords > kRedWords ? kSelWords : kRedWords];
  const int sel_blocks = (a.T + 3) / 4;
  if ((int)blockIdx.x >= sel_blocks) {
    shared_gate_up_tile<CPW>(sh, blockIdx.x - sel_blocks, reinterpret_cast<glm_f32x4 *>(lds));
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = blockIdx.x * 4 + wave;
  if (t >= a.T) return;  // wave-uniform; the selection synchronises one wave only
  int *sel = reinterpret_cast<int *>(lds + 4 * (64 * EPL + 256)) + wave * 64;
  select_token<EPL>(a.logits + (size_t)t * a.E, a.bias, a.E, a.k, a.n_group, a.topk_group,
                    a.norm, a.scale, a.weights + (size_t)t * a.k, a.indices + (size_t)t * a.k, sel,
                    lds + wave * (64 * EPL + 256), lane);
}

// One block: selection for every token, then the dispatch of its P pairs.
template <int EPL, int CPW_S>
__global__ __launch_bounds__(kRouteThreads) void select_dispatch_kernel(RouteArgs a,
                                                                        SharedArgs sh) {
  extern __shared__ int lds[];
  __shared__ int s_tmp[4];
  if (blockIdx.x > 0) {
    shared_down_tile<CPW_S>(sh, blockIdx.x - 1, reinterpret_cast<uint16_t *>(lds));
    return;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int T = a.T, E = a.E, k = a.k;
  const int P = T * k;
  int *s_idx = lds;                       // [P]
  int *cnt = s_idx + kMaxFusedPairs;      // [E]
  int *off = cnt + kFusedMaxE;            // [E]
  int *s_active = off + kFusedMaxE;       // [E]
  uint32_t *bits = (uint32_t *)(s_active + kFusedMaxE);  // [E][16]
  float *wave_scratch = (float *)(bits + kFusedMaxE * 16) + wave * (64 * EPL + 256);

  // many tokens: the selection ran one wave per token in an earlier kernel;
  // its indices (P <= 512: two per thread) are loaded before the LDS is
  // cleared, so the memory round trip overlaps the clearing
  constexpr int kPairsPerThread = kMaxFusedPairs / kRouteThreads;
  int pre[kPairsPerThread];
  if (a.presel) {
#pragma unroll
    for (int u = 0; u < kPairsPerThread; ++u) {
      const int p = threadIdx.x + kRouteThreads * u;
      pre[u] = p < P ? (int)a.indices[p] : 0;
    }
  }
  for (int i = threadIdx.x; i < E; i += kRouteThreads) cnt[i] = 0;
  for (int i = threadIdx.x; i < E * 16; i += kRouteThreads) bits[i] = 0;
  if (a.presel) {
#pragma unroll
    for (int u = 0; u < kPairsPerThread; ++u) {
      const int p = threadIdx.x + kRouteThreads * u;
      if (p < P) s_idx[p] = pre[u];
    }
  } else {
    // top-k per token (wave w: tokens w, w+4, ...)
    for (int t = wave; t < T; t += 4)
      select_token<EPL>(a.logits + (size_t)t * E, a.bias, E, k, a.n_group, a.topk_group, a.norm,
                        a.scale, a.weights + (size_t)t * k, a.indices + (size_t)t * k,
                        s_idx + t * k, wave_scratch, lane);
  }
  __syncthreads();

  for (int p = threadIdx.x; p < P; p += kRouteThreads) {
    const int ee = s_idx[p];
    atomicAdd(&cnt[ee], 1);
    atomicOr(&bits[ee * 16 + (p >> 5)], 1u << (p & 31));
  }
  __syncthreads();
  const int per = (E + kRouteThreads - 1) / kRouteThreads;  // experts per thread (<= 2)
  int local = 0, local_act = 0;
  for (int i = 0; i < per; ++i) {
    const int ee = threadIdx.x * per + i;
    if (ee < E) {
      local += cnt[ee];
      local_act += cnt[ee] > 0;
    }
  }
  int tot = 0, tot_act = 0;
  const int base = scan256(local, s_tmp, &tot);
  const int base_act = scan256(local_act, s_tmp, &tot_act);
  {
    int run = base, run_act = base_act;
    for (int i = 0; i < per; ++i) {
      const int ee = threadIdx.x * per + i;
      if (ee < E) {
        off[ee] = run;
        a.offsets[ee] = run;
        a.counts[ee] = cnt[ee];
        if (cnt[ee] > 0) {
          s_active[run_act] = ee;
          ++run_act;
        }
        run += cnt[ee];
      }
    }
  }
  if (threadIdx.x == 0) {
    a.offsets[E] = tot;
    a.num_active[0] = tot_act;
    a.status[0] = 0;
  }
  __syncthreads();
  // The work slots go busiest expert first (ties by expert id): the routed
  // kernels' workgroups run in slot order, and a popular expert's tiles, which
  // loop over several token batches, would otherwise start last and set the
  // launch's tail.  `active` stays ascending.  Slot of active expert u = the
  // number of keys above its own, key(v) = count(v) * 1024 + 1023 - v (all
  // distinct; the pad keys up to a multiple of 4 are -1, below every key).
  int *key = reinterpret_cast<int *>(bits + kFusedMaxE * 16);  // [E] (selection scratch)
  const int nkey = (tot_act + 3) & ~3;
  for (int u = threadIdx.x; u < nkey; u += kRouteThreads)
    key[u] = u < tot_act ? cnt[s_active[u]] * 1024 + 1023 - u : -1;
  __syncthreads();
  for (int u = threadIdx.x; u < E; u += kRouteThreads) {
    if (u < tot_act) {
      const int ee = s_active[u];
      const int c = cnt[ee];
      const int ku = key[u];
      int slot = 0;
      for (int v = 0; v < nkey; v += 4) {
        const int4 kv = *reinterpret_cast<const int4 *>(key + v);
        slot += (kv.x > ku) + (kv.y > ku) + (kv.z > ku) + (kv.w > ku);
      }
      a.active[u] = ee;
      a.work[slot] = make_int4(ee, off[ee], c, 0);
    } else {
      a.active[u] = -1;
      a.work[u] = make_int4(-1, 0, 0, 0);
    }
  }
  for (int p = threadIdx.x; p < P; p += kRouteThreads) {
    const int ee = s_idx[p];
    const uint32_t *row = bits + ee * 16;
    int r = 0;
    const int word = p >> 5;
    for (int w = 0; w < word; ++w) r += __popc(row[w]);
    r += __popc(row[word] & ((1u << (p & 31)) - 1u));
    const int pos = off[ee] + r;
    a.perm[pos] = p;
    a.inv[p] = pos;
    a.pair_token[pos] = p / k;
  }
}

// ---------------------------------------------------------------------------
// Gate/up: grid (row tiles, [1 +] slots).  With a shared expert, grid row 0
// holds its bf16 tiles (all T tokens) and row 1 + u the routed expert of work
// slot u (MXFP4); otherwise row u is work slot u.
// Four waves split K; wave 0 reduces and applies SwiGLU.
// ---------------------------------------------------------------------------
struct GateUpArgs {
  const uint16_t *x;
  const int32_t *pair_token;
  const int4 *work;
  int slots;
  const uint8_t *gw, *gs, *uw, *us;
  long long w_stride, s_stride;
  int I, d;
  uint16_t *h;  // [P][I]
  float limit;
  int shared_blocks;  // leading blocks that are the shared expert's gate/up tiles
};

// Routed gate/up: block b = (work slot b / (I/16), 16-row tile); 4 waves split
// d.  The weights are loaded once; the expert's tokens go through in batches
// of 16 (the MFMA's columns), each lane column reading its token's row from
// global memory.  With the shared expert riding along, the first
// a.shared_blocks blocks are its full-K gate/up tiles (shared_gate_up_tile).
template <int CPW>
__global__ __launch_bounds__(256) void decode_gate_up_kernel(GateUpArgs a, SharedArgs sh) {
  __shared__ glm_f32x4 red[3 * 2 * 64];
  if ((int)blockIdx.x < a.shared_blocks) {
    shared_gate_up_tile<CPW>(sh, blockIdx.x, red);
    return;
  }
  const int blk = (int)blockIdx.x - a.shared_blocks;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int d = a.d;
  const int tiles = a.I / 16;
  const int4 wk = a.work[blk / tiles];
  const int row0 = (blk % tiles) * 16;
  const int e = wk.x, base = wk.y, n = wk.z;
  if (e < 0 || n <= 0) return;
  const int kbase = wave * CPW * 128;
  const uint8_t *wtile[2] = {tile_lane_ptr(a.gw + e * a.w_stride, row0, d, lane),
                             tile_lane_ptr(a.uw + e * a.w_stride, row0, d, lane)};
  const uint8_t *srow[2] = {a.gs + e * a.s_stride + (size_t)(row0 + r) * (d / 32),
                            a.us + e * a.s_stride + (size_t)(row0 + r) * (d / 32)};
  // the weight stream once for all token batches; lane column r reads its
  // token's row straight from global memory (L2-resident), in flight with
  // the weights
  WaveWeights<FMT_MXFP4, 2, CPW> ww;
  load_wave_weights<FMT_MXFP4, 2, CPW>(ww, wtile, srow, kbase, q);
  for (int p0 = 0; p0 < n; p0 += 16) {
    const int rows = min(16, n - p0);
    // Opaque to the compiler per batch: the weights' conversion stays inside
    // the loop, after this batch's activation loads are issued, instead of
    // being hoisted in front of it (that would pin 128 registers of
    // converted weights and serialise the activation loads).
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int c = 0; c < CPW; ++c) asm volatile("" : "+v"(ww.w[p][c].c));
    const uint16_t *act = a.x + (size_t)a.pair_token[base + p0 + min(r, rows - 1)] * d;
    glm_f32x4 acc[2] = {glm_f32x4{0.f, 0.f, 0.f, 0.f}, glm_f32x4{0.f, 0.f, 0.f, 0.f}};
    mma_wave_weights<FMT_MXFP4, 2, CPW>(ww, kbase, q, act, acc);
    if (ksplit_reduce<2>(acc, red, wave, 4, lane) && r < rows) {
      uint32_t o[4];
#pragma unroll
      for (int m = 0; m < 4; ++m)
        o[m] = f32_to_bf16(limited_swiglu(bf16_round(acc[0][m]), bf16_round(acc[1][m]), a.limit));
      store_rows4(a.h + (size_t)(base + p0 + r) * a.I + row0 + 4 * q, o);
    }
  }
}

constexpr int kDownStageRows = 16;  // h rows per LDS batch (the MFMA's 16 columns)

struct DownArgs {
  const uint16_t *h;
  const int4 *work;
  int slots;
  const uint8_t *dw, *ds;
  long long w_stride, s_stride;
  int I, d;
  uint16_t *y;  // [P][d]
  int shared_blocks;  // leading blocks that are the shared expert's down tiles
};

// Routed down: block b = (work slot b / (d/64), 64-row tile); each wave owns
// 16 output rows over the full K = I.  The weights are loaded once; the
// slot's h rows go through in batches of 16, staged in LDS (all four waves
// read every row).  With the shared expert riding along, the first
// a.shared_blocks blocks are its down tiles over the full-K gate/up tiles'
// bf16 activations (shared_down_tile; no LDS).
template <int CPW_R, int CPW_S>
__global__ __launch_bounds__(256) void decode_down_kernel(DownArgs a, SharedArgs sh) {
  extern __shared__ __attribute__((aligned(16))) uint16_t s_x[];  // [16][lds_row_stride(I)]
  if ((int)blockIdx.x < a.shared_blocks) {
    shared_down_tile<CPW_S>(sh, blockIdx.x, s_x);
    return;
  }
  const int blk = (int)blockIdx.x - a.shared_blocks;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int d = a.d;
  const int tiles = d / 64;
  const int4 wk = a.work[blk / tiles];
  const int row0 = (blk % tiles) * 64 + wave * 16;
  const int e = wk.x, base = wk.y, n = wk.z;
  if (e < 0 || n <= 0) return;
  const uint8_t *wtile[1] = {tile_lane_ptr(a.dw + e * a.w_stride, row0, a.I, lane)};
  const uint8_t *srow[1] = {a.ds + e * a.s_stride + (size_t)(row0 + r) * (a.I / 32)};
  WaveWeights<FMT_MXFP4, 1, CPW_R> ww;  // loaded once for all token batches
  load_wave_weights<FMT_MXFP4, 1, CPW_R>(ww, wtile, srow, 0, q);
  for (int p0 = 0; p0 < n; p0 += kDownStageRows) {
    const int rows = min(kDownStageRows, n - p0);
    if constexpr (CPW_R > 8) {
      // Opaque per batch: converted weights of 16 chunks would pin 256
      // registers (one wave per SIMD) if hoisted out of the batch loop.
#pragma unroll
      for (int c = 0; c < CPW_R; ++c) asm volatile("" : "+v"(ww.w[0][c].c));
    }
    if (p0 > 0) __syncthreads();
    stage_rows(s_x, a.h + (size_t)(base + p0) * a.I, nullptr, rows, a.I);
    __syncthreads();
    glm_f32x4 acc[1] = {glm_f32x4{0.f, 0.f, 0.f, 0.f}};
    mma_wave_weights_lds<FMT_MXFP4, 1, CPW_R>(ww, 0, q,
                                              s_x + min(r, rows - 1) * lds_row_stride(a.I), acc);
    if (r < rows) {
      uint32_t o[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) o[m] = f32_to_bf16(acc[0][m]);
      store_rows4(a.y + (size_t)(base + p0 + r) * d + row0 + 4 * q, o);
    }
  }
}

// ---------------------------------------------------------------------------
// Few-token path: token-major selection + gate/up, then down + combine.
// ---------------------------------------------------------------------------
constexpr int kPairMaxT = 4;
constexpr int kPairMaxK = 8;
// 16-byte pieces of h per thread in down_combine_kernel: k*I/8 pieces over
// 64*max(k, 4) threads is at most I/512 = CPW_R/4 (I = 128 CPW_R)
__host__ __device__ constexpr int h_pieces(int cpw_r) { return cpw_r < 4 ? 1 : (cpw_r + 3) / 4; }

struct PairArgs {
  const float *logits, *bias;
  int T, E, k, n_group, topk_group, norm;
  float scale;
  float *weights;     // [T][k]
  uint32_t *indices;  // [T][k]
  const uint16_t *x;
  const uint8_t *gw, *gs, *uw, *us;
  long long w_stride, s_stride;
  int d, I;
  uint16_t *h;  // [T*k][I] in pair order
  float limit;
  int routed_blocks;
  int tpb;  // 16-row tiles of one pair per routed block (consecutive)
  // ScaleX Mode-B scale rows (SX kernels; gs and us unused): expert e's row
  // at sx + e * sx_stride
  const uint8_t *sx;
  long long sx_stride;
};

// LDS bytes of select_gate_up_kernel: the token row, then each of the four
// waves' selection scratch and choice; shared down tiles reuse the area for
// their activations.
__host__ __device__ constexpr size_t pair_gate_up_lds_bytes(int d, int EPL) {
  return (size_t)lds_row_stride(d) * 2 + (size_t)4 * (64 * EPL + 256 + 64) * 4;
}

// LDS bytes of the decoded scale rows of an SX select_gate_up block: the
// gate and the up rows of its tiles.
__host__ __device__ constexpr size_t pair_gate_up_sx_bytes(int d, int tpb) {
  return (size_t)2 * 16 * tpb * (d / 32);
}

// Four waves per SIMD (at most 128 registers, no spills): at the real expert
// geometry the routed and the shared-down blocks of one launch are then all
// resident at once.
template <int EPL, int CPW, int CPW_S, bool SX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void select_gate_up_kernel(PairArgs a, SharedArgs sh) {
  extern __shared__ __attribute__((aligned(16))) uint16_t s_dyn[];
  __shared__ glm_f32x4 red[3 * 2 * 64];
  if ((int)blockIdx.x >= a.routed_blocks) {
    shared_down_tile<CPW_S>(sh, blockIdx.x - a.routed_blocks, s_dyn);
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int d = a.d, k = a.k, E = a.E;
  const int groups = a.I / 16 / a.tpb;     // blocks per pair
  const int tile0 = (blockIdx.x % groups) * a.tpb;
  const int pr = blockIdx.x / groups;  // pair t*k + j
  const int t = pr / k, j = pr % k;
  const bool first = j == 0 && tile0 == 0;  // one block per token publishes the route
  // Each wave stages the K range of token t's row that it multiplies and
  // selects the token's experts itself (moe.py:39-62; every wave reaches the
  // same choice), so no block barrier stands between the route and the
  // weight loads.  Wave 0 of one block per token publishes the route.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  uint16_t *s_x = s_dyn;  // token t's row
  // the wave's K range of the row goes to registers first and to LDS after
  // the selection, whose logit and bias loads then share its round trip
  constexpr int kRowPieces = (CPW * 16 + 63) / 64;
  glm_u32x4 xrow[kRowPieces];
  {
    const glm_u32x4 *src = reinterpret_cast<const glm_u32x4 *>(a.x + (size_t)t * d + wv * CPW * 128);
#pragma unroll
    for (int u = 0; u < kRowPieces; ++u) xrow[u] = src[min(lane + 64 * u, CPW * 16 - 1)];
  }
  float *scratch = reinterpret_cast<float *>(s_dyn + lds_row_stride(d)) + wv * (64 * EPL + 256 + 64);
  int *s_selw = reinterpret_cast<int *>(scratch + 64 * EPL + 256);
  const bool publish = first && wv == 0;
  select_token<EPL>(a.logits + (size_t)t * E, a.bias, E, k, a.n_group, a.topk_group, a.norm,
                    a.scale, publish ? a.weights + (size_t)t * k : nullptr,
                    publish ? a.indices + (size_t)t * k : nullptr, s_selw, scratch, lane);
  {
    glm_u32x4 *dst = reinterpret_cast<glm_u32x4 *>(s_x + wv * CPW * 128);
#pragma unroll
    for (int u = 0; u < kRowPieces; ++u)
      if (lane + 64 * u < CPW * 16) dst[lane + 64 * u] = xrow[u];
  }
  wave_lds_sync();  // the staged row and the choice, for this wave
  const long long e = s_selw[j];
  const int kbase = wv * CPW * 128;
  // the block's tiles in turn; the next tile's weights are issued as soon as
  // the MFMAs have consumed this tile's registers, so the wave streams them
  // back to back and the route above is paid once per block
  const uint8_t *gw = a.gw + e * a.w_stride, *uw = a.uw + e * a.w_stride;
  const uint8_t *gs = a.gs + e * a.s_stride, *us = a.us + e * a.s_stride;
  WaveWeights<FMT_MXFP4, 2, CPW> ww;
  // SX: the gate and the up scale rows of the block's tiles, decoded from the
  // expert's Mode-B row into LDS by the whole block while the first tile's
  // weights are in flight (gate scales at 16 r' G, up at (16 tpb + 16 r') G)
  const int G = d / 32, nsx = 16 * a.tpb;
  uint8_t *s_sc = reinterpret_cast<uint8_t *>(s_dyn) + pair_gate_up_lds_bytes(d, EPL);
  {
    const int row = tile0 * 16 + r;
    const uint8_t *wtile[2] = {tile_lane_ptr(gw, tile0 * 16, d, lane),
                               tile_lane_ptr(uw, tile0 * 16, d, lane)};
    if constexpr (SX) {
      load_wave_chunks<FMT_MXFP4, 2, CPW>(ww, wtile, kbase, q);
      const ScalexRow hx = scalex_row(a.sx + e * a.sx_stride, scalex_dir_bytes(3 * a.I * (a.d / 32)));
      const uint32_t s0[2] = {(uint32_t)(tile0 * 16 * G), (uint32_t)((2 * a.I + tile0 * 16) * G)};
      uint8_t *const dst[2] = {s_sc, s_sc + nsx * G};
      scalex_decode<2>(hx, s0, (uint32_t)(nsx * G), dst, (int)threadIdx.x, 256,
                       [] { __syncthreads(); });
      __syncthreads();
      const uint8_t *srow[2] = {s_sc + r * G, s_sc + (nsx + r) * G};
      wave_scales_from_lds<FMT_MXFP4, 2, CPW>(ww, srow, kbase, q);
    } else {
      const uint8_t *srow[2] = {gs + (size_t)row * (d / 32), us + (size_t)row * (d / 32)};
      load_wave_weights<FMT_MXFP4, 2, CPW>(ww, wtile, srow, kbase, q);
    }
  }
  for (int ti = 0; ti < a.tpb; ++ti) {
    const int row0 = (tile0 + ti) * 16;
    glm_f32x4 acc[2] = {glm_f32x4{0.f, 0.f, 0.f, 0.f}, glm_f32x4{0.f, 0.f, 0.f, 0.f}};
    mma_wave_weights_lds<FMT_MXFP4, 2, CPW>(ww, kbase, q, s_x, acc);  // column 0 is stored
    if (ti + 1 < a.tpb) {
      const int row = row0 + 16 + r;
      const uint8_t *wtile[2] = {tile_lane_ptr(gw, row0 + 16, d, lane),
                                 tile_lane_ptr(uw, row0 + 16, d, lane)};
      if constexpr (SX) {
        load_wave_chunks<FMT_MXFP4, 2, CPW>(ww, wtile, kbase, q);
        const int rr = (ti + 1) * 16 + r;
        const uint8_t *srow[2] = {s_sc + rr * G, s_sc + (nsx + rr) * G};
        wave_scales_from_lds<FMT_MXFP4, 2, CPW>(ww, srow, kbase, q);
      } else {
        const uint8_t *srow[2] = {gs + (size_t)row * (d / 32), us + (size_t)row * (d / 32)};
        load_wave_weights<FMT_MXFP4, 2, CPW>(ww, wtile, srow, kbase, q);
      }
    }
    if (ksplit_reduce<2>(acc, red, wave, 4, lane) && r == 0) {
      uint32_t o[4];
#pragma unroll
      for (int m = 0; m < 4; ++m)
        o[m] = f32_to_bf16(limited_swiglu(bf16_round(acc[0][m]), bf16_round(acc[1][m]), a.limit));
      store_rows4(a.h + (size_t)pr * a.I + row0 + 4 * q, o);
    }
  }
}

// 16-row tiles per routed block of select_gate_up_kernel: one while the grid
// is small (up to 16 pairs x 48 tiles, one or two tokens at I 768); with
// more tiles each block streams several consecutive tiles of its pair, up to
// four, so the token row + selection before the first weight load is paid
// once per block, not once per tile (four at the real expert geometry, 16
// pairs x 128 tiles, where eight measured 60.9 against 59.6 us).  Two tiles
// at 16 pairs x 48 tiles measured within the run-to-run spread of one
// (20.91 against 20.99 us per step, interleaved on one box) and made the
// kernel itself 4 % slower.
static int pair_tiles_per_block(int pairs, int I) {
  const int tiles = I / 16;
  int tpb = 1;
  while (tpb < 4 && (long long)pairs * tiles / tpb > 768 && tiles % (2 * tpb) == 0) tpb *= 2;
  return tpb;
}

struct PairDownArgs {
  const uint16_t *h;  // [T*k][I] in pair order
  const float *weights;
  const uint32_t *indices;
  const uint8_t *dw, *ds;
  long long w_stride, s_stride;
  int T, k, I, d;
  const uint16_t *shared;      // bf16 shared output [T][d], or
  const float *shared_parts;   // its f32 K-range partial sums [nparts][T][d], or neither
  int nparts;
  float *out;  // [T][d] f32
  // optional hyper_residual of the decoder FFN site (hc_out != nullptr):
  // hc_out[t][j] = post[t][j] out[t] + sum_i comb[t][i][j] hc_res[t][i]
  const float *hc_res, *hc_post, *hc_comb;  // [T][hc][d], [T][hc], [T][hc][hc]
  float *hc_out;                            // [T][hc][d]
  int hc, hc_bf16;                          // hc_bf16: bf16 streams (GLM_HC_BF16_STREAMS)
  int tpb;  // 16-row tiles of d per block (consecutive)
  // ScaleX Mode-B scale rows (SX kernels; ds unused)
  const uint8_t *sx;
  long long sx_stride;
};

constexpr int kPairMaxHc = 8;
constexpr int kPairMaxParts = 8;    // shared down partial sums (Is <= 2048)
constexpr int kPairMaxCols = 64;    // output columns of a down_combine block (tpb <= 4)

// Down projection of all k experts of one token on 16 rows of d, merged in
// the combine's order: out = sum_j f32(bf16(y_j)) * w_j (sequential j, no
// contraction) + shared, where shared = bf16 of its partial sums added in
// order.  Wave j (of max(k, 4)) owns expert j over the full K = I.
template <int CPW_R, bool SX>
__global__ __launch_bounds__(512) void down_combine_kernel(PairDownArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) uint16_t s_h[];  // [k][lds_row_stride(I)]
  __shared__ float s_p[kPairMaxK][16];
  __shared__ float s_shv[kPairMaxCols];              // shared contribution per column
  __shared__ float s_rv[kPairMaxHc][kPairMaxCols];   // residual streams per column
  __shared__ float s_hc[kPairMaxHc + kPairMaxHc * kPairMaxHc];
  const int lane = threadIdx.x & 63;
  const int j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int k = a.k, d = a.d, I = a.I;
  const int groups = d / 16 / a.tpb;  // blocks per token
  const int t = blockIdx.x / groups;
  const int tile0 = (blockIdx.x % groups) * a.tpb;
  const int ncol = 16 * a.tpb;  // the block's output columns tile0 * 16 + [0, ncol)
  const int hc = a.hc;
  const bool has_shared = a.shared_parts != nullptr || a.shared != nullptr;
  // The loads go out in this order, the same in every wave and on no
  // branch, so that every wait covers exactly what it needs (a register whose
  // load is pending cannot be merged at a branch join without a full wait):
  // the epilogue's values of the block's columns, one column per lane (shared
  // contribution, residual streams, the FFN site's gates; inputs that are
  // absent read the output row instead, in bounds and unused), the route, the
  // h rows, then the first tile's weights, whose addresses wait only for the
  // route.  Waves past k mirror expert k - 1 and store nothing.
  const int cl = tile0 * 16 + min(lane, ncol - 1);
  const float *spb = a.shared_parts != nullptr ? a.shared_parts : a.out;
  const int np = a.shared_parts != nullptr ? a.nparts : 1;
  float sp[kPairMaxParts];
#pragma unroll
  for (int qq = 0; qq < kPairMaxParts; ++qq)
    sp[qq] = spb[((size_t)min(qq, np - 1) * a.T + t) * d + cl];
  const uint16_t *sbf = a.shared != nullptr ? a.shared : reinterpret_cast<const uint16_t *>(a.out);
  const uint16_t sb = sbf[(size_t)t * d + cl];
  const bool fuse_hc = a.hc_out != nullptr;
  const int hcc = fuse_hc ? hc : 1;
  const float *rvb = fuse_hc ? a.hc_res : a.out;
  float rv[kPairMaxHc];
#pragma unroll
  for (int i = 0; i < kPairMaxHc; ++i) rv[i] = rvb[((size_t)t * hcc + min(i, hcc - 1)) * d + cl];
  // gates: hc post values, then hc x hc comb values (<= 72: entries lane, lane + 64)
  const float *postb = fuse_hc ? a.hc_post : a.out, *combb = fuse_hc ? a.hc_comb : a.out;
  float gate[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int i = min(lane + 64 * g, hcc + hcc * hcc - 1);
    gate[g] = i < hcc ? postb[(size_t)t * hcc + i] : combb[(size_t)t * hcc * hcc + i - hcc];
  }
  const int jr = min(j, k - 1);
  const long long e = a.indices[(size_t)t * k + jr];
  const float wj = a.weights[(size_t)t * k + jr];
  const int per_row = I / 8, nh = k * per_row;  // 16-byte pieces of the k rows of h
  const uint16_t *hsrc = a.h + (size_t)t * k * I;
  constexpr int kHP = h_pieces(CPW_R);
  glm_u32x4 hv[kHP];
#pragma unroll
  for (int u = 0; u < kHP; ++u) {
    const int i = min((int)threadIdx.x + (int)blockDim.x * u, nh - 1);
    hv[u] = *reinterpret_cast<const glm_u32x4 *>(hsrc + (size_t)i * 8);
  }
  const uint8_t *dw = a.dw + e * a.w_stride, *ds = a.ds + e * a.s_stride;
  WaveWeights<FMT_MXFP4, 1, CPW_R> ww;
  // SX: wave j decodes the down scale rows of its expert for the block's
  // tiles into its own LDS area (after h), while the first tile's weights
  // are in flight
  const int Gi = I / 32, nsx = 16 * a.tpb;
  uint8_t *s_sc = reinterpret_cast<uint8_t *>(s_h) + (size_t)k * lds_row_stride(I) * 2 +
                  (size_t)jr * nsx * Gi;
  {
    const int row = tile0 * 16 + r;
    const uint8_t *wtile[1] = {tile_lane_ptr(dw, tile0 * 16, I, lane)};
    if constexpr (SX) {
      load_wave_chunks<FMT_MXFP4, 1, CPW_R>(ww, wtile, 0, q);
    } else {
      const uint8_t *srow[1] = {ds + (size_t)row * (I / 32)};
      load_wave_weights<FMT_MXFP4, 1, CPW_R>(ww, wtile, srow, 0, q);
    }
  }
  // the epilogue's values to LDS (the shared partial sums added in order)
  if (j == 0 && lane < ncol) {
    float v = sp[0];
#pragma unroll
    for (int qq = 1; qq < kPairMaxParts; ++qq) v = qq < np ? v + sp[qq] : v;
    s_shv[lane] = a.shared_parts != nullptr ? bf16_round(v) : bf16_to_f32(sb);
#pragma unroll
    for (int i = 0; i < kPairMaxHc; ++i) s_rv[i][lane] = i < hc ? rv[i] : 0.0f;
  } else if (j == 1 && fuse_hc) {
#pragma unroll
    for (int g = 0; g < 2; ++g)
      if (lane + 64 * g < hc + hc * hc) s_hc[lane + 64 * g] = gate[g];
  }
#pragma unroll
  for (int u = 0; u < kHP; ++u) {
    const int i = (int)threadIdx.x + (int)blockDim.x * u;
    if (i < nh)
      *reinterpret_cast<glm_u32x4 *>(s_h + (i / per_row) * lds_row_stride(I) + (i % per_row) * 8) = hv[u];
  }
  if constexpr (SX) {
    if (j < k) {
      const ScalexRow hx = scalex_row(a.sx + e * a.sx_stride, scalex_dir_bytes(3 * a.I * (a.d / 32)));
      // the down scales follow the gate's I x d/32 in the expert's stream
      const uint32_t s0[1] = {(uint32_t)(I * (d / 32) + tile0 * 16 * Gi)};
      uint8_t *const dst[1] = {s_sc};
      scalex_decode<1>(hx, s0, (uint32_t)(nsx * Gi), dst, lane, 64, [] { wave_lds_sync(); });
    }
    wave_lds_sync();
    const uint8_t *srow[1] = {s_sc + r * Gi};
    wave_scales_from_lds<FMT_MXFP4, 1, CPW_R>(ww, srow, 0, q);
  }
  // the block's 16-row tiles in turn; the next tile's weights are issued as
  // soon as the MFMAs have consumed this tile's registers
  for (int ti = 0; ti < a.tpb; ++ti) {
    const int row0 = (tile0 + ti) * 16;
    __syncthreads();  // h and the epilogue's values in LDS (first tile); s_p free again (later tiles)
    glm_f32x4 acc[1] = {glm_f32x4{0.f, 0.f, 0.f, 0.f}};
    if constexpr (!SX) {
      const int row = row0 + 16 + r;
      const uint8_t *wtile[1] = {tile_lane_ptr(dw, row0 + 16, I, lane)};
      const uint8_t *srow[1] = {ds + (size_t)row * (I / 32)};
      mma_wave_weights_lds_roll<FMT_MXFP4, 1, CPW_R>(ww, 0, q, s_h + jr * lds_row_stride(I), acc,
                                                     ti + 1 < a.tpb, wtile, srow);
    } else {
      mma_wave_weights_lds<FMT_MXFP4, 1, CPW_R>(ww, 0, q, s_h + jr * lds_row_stride(I),
                                                acc);  // column 0 is stored
      if (ti + 1 < a.tpb) {
        const uint8_t *wtile[1] = {tile_lane_ptr(dw, row0 + 16, I, lane)};
        load_wave_chunks<FMT_MXFP4, 1, CPW_R>(ww, wtile, 0, q);
        const uint8_t *srow[1] = {s_sc + ((ti + 1) * 16 + r) * Gi};
        wave_scales_from_lds<FMT_MXFP4, 1, CPW_R>(ww, srow, 0, q);
      }
    }
    if (j < k && r == 0) {
#pragma unroll
      for (int m = 0; m < 4; ++m) s_p[j][4 * q + m] = bf16_round(acc[0][m]) * wj;
    }
    __syncthreads();
    if (threadIdx.x < 16) {
      const int cc = ti * 16 + threadIdx.x;  // column row0 + threadIdx.x among the block's
      const int c = row0 + threadIdx.x;
      float o = 0.0f;
      for (int jj = 0; jj < k; ++jj) o = o + s_p[jj][threadIdx.x];
      if (has_shared) o = o + s_shv[cc];
      a.out[(size_t)t * d + c] = o;
      if (a.hc_out != nullptr) {
        // hyper_residual (mhc.py:51-60): the placement and the mixing sum
        // rounded as separate operations; bf16 streams round post, comb and
        // the mixing sum to bf16
        for (int jj = 0; jj < hc; ++jj) {
          float pj = s_hc[jj];
          if (a.hc_bf16) pj = bf16_round(pj);
          float m = 0.0f;
#pragma unroll
          for (int i = 0; i < kPairMaxHc; ++i) {
            if (i < hc) {
              float w = s_hc[hc + i * hc + jj];
              if (a.hc_bf16) w = bf16_round(w);
              m = m + w * s_rv[i][cc];
            }
          }
          if (a.hc_bf16) m = bf16_round(m);
          a.hc_out[((size_t)t * hc + jj) * d + c] = pj * o + m;
        }
      }
    }
  }
}

// zero-fill (workspace initialisation)
__global__ void fill_zero_kernel(uint32_t *p, long long n) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    p[i] = 0;
}

}  // namespace glm

using namespace glm;

size_t glm_select_dispatch_lds_bytes(int EPL) {
  return (size_t)(kMaxFusedPairs + 3 * kFusedMaxE + 16 * kFusedMaxE) * 4 +
         (size_t)4 * (64 * EPL + 256) * 4;
}

// Whether the decode kernels cover this layer shape: gate/up waves take d/512
// chunks of 128 (d / 4 per wave), down waves the whole K = I in I/128 chunks
// (16 at the real expert geometry, I 2048); the shared expert's down tiles
// take 1 or 2 chunks per K range.
static bool chunk_count_ok(int c) { return c == 1 || c == 2 || c == 4 || c == 6 || c == 8; }
static bool down_chunks_ok(int c) { return chunk_count_ok(c) || c == 16; }
static bool shared_chunks_ok(int c) { return c == 1 || (c % 2 == 0 && c <= 16); }

bool glm_decode_gate_up_supported(int d, int I) {
  return d % 512 == 0 && d / 512 >= 2 && chunk_count_ok(d / 512) && I % 16 == 0;
}

bool glm_decode_down_supported(int I, int d) {
  return I % 128 == 0 && down_chunks_ok(I / 128) && d % 64 == 0;
}

bool glm_decode_path_supported(int T, int d, int E, int k, int I, int Is) {
  if (T < 1 || T > 64 || (long long)T * k > kMaxFusedPairs || E > kFusedMaxE) return false;
  // gate/up: 4 waves x CPW chunks of 128 over d; down: 64-row tiles of d
  if (d % 512 != 0 || !chunk_count_ok(d / 512) || d / 512 < 2) return false;
  if (I % 128 != 0 || !down_chunks_ok(I / 128)) return false;
  if (Is > 0 && (Is % 128 != 0 || !shared_chunks_ok(Is / 128))) return false;
  return true;
}

// Shared-expert splits: gate/up K in d/512 ranges when T <= 8 (one 128-wide
// chunk per wave), else full-K tiles; down K in ranges of 2 chunks (1 if Is == 128).
int glm_decode_shared_skq(int T, int d) { return T <= 8 ? d / 512 : 1; }
int glm_decode_shared_cpws(int Is) { return Is / 128 == 1 ? 1 : 2; }
int glm_decode_shared_skd(int Is) { return Is / 128 / glm_decode_shared_cpws(Is); }

static SharedArgs make_shared_args(const uint16_t *x, int T, int d, const uint16_t *sg,
                                   const uint16_t *su, const uint16_t *sd, int Is, float *gp,
                                   float *up, uint16_t *hs, float *yp, float limit) {
  SharedArgs sh{};
  sh.x = x;
  sh.sg = reinterpret_cast<const uint8_t *>(sg);
  sh.su = reinterpret_cast<const uint8_t *>(su);
  sh.sd = reinterpret_cast<const uint8_t *>(sd);
  sh.T = T;
  sh.d = d;
  sh.Is = sg ? Is : 0;
  sh.skq = glm_decode_shared_skq(T, d);
  sh.skd = sg ? glm_decode_shared_skd(Is) : 1;
  // full-K tiles (skq == 1) split the tokens into groups of 16 across blocks
  const int tgroups = sh.skq > 1 ? 1 : (T + 15) / 16;
  sh.gu_blocks = sg ? (Is / 16) * sh.skq * tgroups : 0;
  sh.dn_blocks = sg ? (d / 64) * sh.skd * tgroups : 0;
  sh.gp = gp;
  sh.up = up;
  sh.hs = hs;
  sh.yp = yp;
  sh.limit = glm_limit_bf16(limit);
  return sh;
}

// Router logits for every token, plus the shared expert's gate/up tiles.
static int launch_route_logits(hipStream_t stream, const RouteArgs &a, const SharedArgs &sh) {
  const int cpw = a.d / 512;
  const dim3 g1((a.logits_done ? 0 : a.E) + sh.gu_blocks);
  if (g1.x == 0) return GLM_OK;
#define GLM_LOGITS(TT)                                                                          \
  switch (cpw) {                                                                                \
    case 2: hipLaunchKernelGGL((route_logits_kernel<TT, 2>), g1, dim3(kRouteThreads), 0, stream, a, sh); break; \
    case 4: hipLaunchKernelGGL((route_logits_kernel<TT, 4>), g1, dim3(kRouteThreads), 0, stream, a, sh); break; \
    case 6: hipLaunchKernelGGL((route_logits_kernel<TT, 6>), g1, dim3(kRouteThreads), 0, stream, a, sh); break; \
    default: hipLaunchKernelGGL((route_logits_kernel<TT, 8>), g1, dim3(kRouteThreads), 0, stream, a, sh); break; \
  }
  // tokens per pass over the expert's router row
  if (a.T <= 2) {
    GLM_LOGITS(2)
  } else if (a.T <= 8) {
    GLM_LOGITS(8)
  } else if (a.T <= 16) {
    GLM_LOGITS(16)
  } else {
    GLM_LOGITS(32)
  }
#undef GLM_LOGITS
  GLM_LAUNCH_CHECK("route_logits_kernel");
  return GLM_OK;
}

int glm_route_decode_launch(hipStream_t stream, const uint16_t *x, int T, int d, const float *w,
                            const float *bias, int E, int k, int n_group, int topk_group,
                            int norm, float scale, float *logits, float *weights,
                            uint32_t *indices, int32_t *counts, int32_t *offsets, int32_t *perm,
                            int32_t *inv, int32_t *pair_token, int32_t *active,
                            int32_t *num_active, int32_t *status, int4 *work,
                            const uint16_t *sg, const uint16_t *su, const uint16_t *sd, int Is,
                            float *gp, float *up, uint16_t *hs, float *yp, float limit) {
  RouteArgs a{x,      w,      bias,   T,   d,          E,      k,          n_group,
              topk_group, norm, scale, logits, weights, indices, counts, offsets,
              perm,   inv,    pair_token, active, num_active, status, work, 0, 0};
  const SharedArgs sh = make_shared_args(x, T, d, sg, su, sd, Is, gp, up, hs, yp, limit);
  int rc;
  const int epl = (E + 63) / 64;
  const int e8 = epl <= 1 ? 1 : (epl <= 2 ? 2 : (epl <= 4 ? 4 : 8));
  if (glm_router_gemm_supported(T, d)) {
    // many tokens: the logits on MFMA, then the selection (one wave per
    // token).  Below 256 tokens with d % 2048 == 0 the shared expert's full-K
    // gate/up tiles run as extra workgroups of the router's launch (router_shared_kernel),
    // otherwise beside the selection.
    SharedArgs sh_sel = sh;
    if (sh.gu_blocks > 0 && sh.skq == 1 && T < 256 && d % 2048 == 0 && d / 2048 <= 2) {
      const int token_tiles = (T + 15) / 16;
      const int router_blocks = token_tiles * ((E + 15) / 16);
      const dim3 g0(router_blocks + sh.gu_blocks);
      if (d / 2048 == 1)
        hipLaunchKernelGGL((router_shared_kernel<1>), g0, dim3(64 * kRouterShWaves), 0, stream, x,
                           w, T, d, E, logits, token_tiles, router_blocks, sh);
      else
        hipLaunchKernelGGL((router_shared_kernel<2>), g0, dim3(64 * kRouterShWaves), 0, stream, x,
                           w, T, d, E, logits, token_tiles, router_blocks, sh);
      GLM_LAUNCH_CHECK("router_shared_kernel");
      sh_sel.gu_blocks = 0;
    } else {
      rc = glm_router_logits_launch(stream, x, T, d, w, E, logits);
      if (rc) return rc;
    }
    a.logits_done = 1;
    a.presel = 1;
    const dim3 g((T + 3) / 4 + sh_sel.gu_blocks);
#define GLM_SS(C)                                                                              \
  switch (e8) {                                                                                \
    case 1: hipLaunchKernelGGL((select_shared_kernel<C, 1>), g, dim3(kRouteThreads), 0, stream, a, sh_sel); break; \
    case 2: hipLaunchKernelGGL((select_shared_kernel<C, 2>), g, dim3(kRouteThreads), 0, stream, a, sh_sel); break; \
    case 4: hipLaunchKernelGGL((select_shared_kernel<C, 4>), g, dim3(kRouteThreads), 0, stream, a, sh_sel); break; \
    default: hipLaunchKernelGGL((select_shared_kernel<C, 8>), g, dim3(kRouteThreads), 0, stream, a, sh_sel); break; \
  }
    switch (d / 512) {
      case 2: GLM_SS(2) break;
      case 4: GLM_SS(4) break;
      case 6: GLM_SS(6) break;
      default: GLM_SS(8) break;
    }
#undef GLM_SS
    GLM_LAUNCH_CHECK("select_shared_kernel");
  } else {
    rc = launch_route_logits(stream, a, sh);
    if (rc) return rc;
    // beyond a few tokens per wave the selection runs one wave per token first
    if (T > 8) {
      rc = glm_router_select_launch(stream, logits, bias, T, E, k, n_group, topk_group, norm,
                                    scale, weights, indices);
      if (rc) return rc;
      a.presel = 1;
    }
  }
  const int cs = sg ? glm_decode_shared_cpws(Is) : 1;
  const size_t lds = std::max(glm_select_dispatch_lds_bytes(e8), (size_t)T * cs * 128 * 2);
  const dim3 g2(1 + sh.dn_blocks);
#define GLM_SEL(EP)                                                                           \
  if (cs == 1)                                                                                \
    hipLaunchKernelGGL((select_dispatch_kernel<EP, 1>), g2, dim3(kRouteThreads), lds, stream, a, sh); \
  else                                                                                        \
    hipLaunchKernelGGL((select_dispatch_kernel<EP, 2>), g2, dim3(kRouteThreads), lds, stream, a, sh)
  if (e8 == 1) GLM_SEL(1);
  else if (e8 == 2) GLM_SEL(2);
  else if (e8 == 4) GLM_SEL(4);
  else GLM_SEL(8);
#undef GLM_SEL
  GLM_LAUNCH_CHECK("select_dispatch_kernel");
  return GLM_OK;
}

// From 16 to 32 tokens (the router on MFMA, full-K shared tiles in one or
// two token groups) the decode path runs the bf16 shared expert's tiles
// inside the routed expert kernels rather than beside the selection and the
// dispatch, which they would otherwise outlast (d 2048, E 128, k 8, I 768:
// 62.5 -> 58.8 us per layer step at 16 tokens, 76.9 -> 74.4 at 32).  At 64
// tokens the four token groups re-read each shared tile four times inside
// the routed stream, which costs more than it saves (92.5 -> 94.0), so there
// the tiles stay beside the selection and the dispatch.
bool glm_decode_shared_in_experts(int T, int d) {
  return glm_router_gemm_supported(T, d) && glm_decode_shared_skq(T, d) == 1 && T <= 32;
}

// Routed gate/up of the decode path; with sg (and su, Is, hs) the shared
// expert's full-K gate/up tiles run as the launch's first blocks and write
// its bf16 activations hs [T][Is] (T > 8 only).
int glm_decode_gate_up_launch(hipStream_t stream, const uint16_t *x, int T, int d, int I, int E,
                              int k, const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                              const uint8_t *us, const int32_t *pair_token, const int4 *work,
                              uint16_t *h, float limit, const uint16_t *sg, const uint16_t *su,
                              int Is, uint16_t *hs) {
  const SharedArgs sh = make_shared_args(x, T, d, sg, su, nullptr, Is, nullptr, nullptr, hs,
                                         nullptr, limit);
  if (sg != nullptr && sh.skq != 1) {
    glm::set_error("decode gate/up: the shared tiles ride along only from 9 tokens on (T=%d)", T);
    return GLM_ERR_UNSUPPORTED_SHAPE;
  }
  GateUpArgs a{};
  a.x = x;
  a.pair_token = pair_token;
  a.work = work;
  a.slots = std::min(E, T * k);
  a.gw = gw;
  a.gs = gs;
  a.uw = uw;
  a.us = us;
  a.w_stride = (long long)I * (d / 2);
  a.s_stride = (long long)I * (d / 32);
  a.I = I;
  a.d = d;
  a.h = h;
  a.limit = glm_limit_bf16(limit);
  a.shared_blocks = sh.gu_blocks;
  const size_t lds = 0;
  const int blocks = a.shared_blocks + a.slots * (I / 16);
  switch (d / 512) {
    case 2: hipLaunchKernelGGL(decode_gate_up_kernel<2>, dim3(blocks), dim3(256), lds, stream, a, sh); break;
    case 4: hipLaunchKernelGGL(decode_gate_up_kernel<4>, dim3(blocks), dim3(256), lds, stream, a, sh); break;
    case 6: hipLaunchKernelGGL(decode_gate_up_kernel<6>, dim3(blocks), dim3(256), lds, stream, a, sh); break;
    case 8: hipLaunchKernelGGL(decode_gate_up_kernel<8>, dim3(blocks), dim3(256), lds, stream, a, sh); break;
    default: glm::set_error("decode gate/up: unsupported d=%d", d); return GLM_ERR_UNSUPPORTED_SHAPE;
  }
  GLM_LAUNCH_CHECK("decode_gate_up_kernel");
  return GLM_OK;
}

// Routed down of the decode path; with sd (and Is, hs, yp) the shared
// expert's down tiles over hs run as the launch's first blocks and write
// their f32 K-range partial sums yp [skd][T][d] (T > 8 only).
int glm_decode_down_launch(hipStream_t stream, const uint16_t *h, int T, int k, int I, int d,
                           int E, const uint8_t *dw, const uint8_t *ds, const int4 *work,
                           uint16_t *y, const uint16_t *sd, int Is, uint16_t *hs, float *yp) {
  // (sd stands in for the gate/up pointers: it only marks the shared expert present)
  const SharedArgs sh = make_shared_args(nullptr, T, d, sd, sd, sd, Is, nullptr, nullptr, hs, yp,
                                         0.0f);
  if (sd != nullptr && sh.skq != 1) {
    glm::set_error("decode down: the shared tiles ride along only from 9 tokens on (T=%d)", T);
    return GLM_ERR_UNSUPPORTED_SHAPE;
  }
  const int cs = sd != nullptr ? glm_decode_shared_cpws(Is) : 1;
  DownArgs a{};
  a.h = h;
  a.work = work;
  a.slots = std::min(E, T * k);
  a.dw = dw;
  a.ds = ds;
  a.w_stride = (long long)d * (I / 2);
  a.s_stride = (long long)d * (I / 32);
  a.I = I;
  a.d = d;
  a.y = y;
  a.shared_blocks = sh.dn_blocks;
  const size_t lds = (size_t)std::min(T * k, kDownStageRows) * lds_row_stride(I) * 2;
  const int blocks = a.shared_blocks + a.slots * (d / 64);
#define GLM_DOWN(CR)                                                                            \
  if (cs == 1)                                                                                  \
    hipLaunchKernelGGL((decode_down_kernel<CR, 1>), dim3(blocks), dim3(256), lds, stream, a, sh); \
  else                                                                                          \
    hipLaunchKernelGGL((decode_down_kernel<CR, 2>), dim3(blocks), dim3(256), lds, stream, a, sh)
  switch (I / 128) {
    case 1: GLM_DOWN(1); break;
    case 2: GLM_DOWN(2); break;
    case 4: GLM_DOWN(4); break;
    case 6: GLM_DOWN(6); break;
    case 8: GLM_DOWN(8); break;
    case 16: GLM_DOWN(16); break;
    default: glm::set_error("decode down: unsupported I=%d", I); return GLM_ERR_UNSUPPORTED_SHAPE;
  }
#undef GLM_DOWN
  GLM_LAUNCH_CHECK("decode_down_kernel");
  return GLM_OK;
}

int glm_fill_zero_launch(hipStream_t stream, void *p, size_t bytes) {
  const long long n = (long long)(bytes / 4);
  if (n == 0) return GLM_OK;
  long long blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     (uint32_t *)p, n);
  GLM_LAUNCH_CHECK("fill_zero_kernel");
  return GLM_OK;
}

// Selection + routed gate/up (+ the shared expert's down tiles of sh, cs
// chunks per tile) of the token-major path.
static int launch_select_gate_up(hipStream_t stream, const PairArgs &a, const SharedArgs &sh,
                                 int cs) {
  const int d = a.d, E = a.E, T = a.T;
  // experts per lane of the selecting wave: E <= 64 * epl
  const int epl = E <= 128 ? 2 : (E <= 256 ? 4 : (E <= 320 ? 5 : 8));
  const bool sx = a.sx != nullptr;
  const size_t lds2 =
      std::max(pair_gate_up_lds_bytes(d, epl) + (sx ? pair_gate_up_sx_bytes(d, a.tpb) : 0),
               (size_t)T * cs * 128 * 2);
  const dim3 g2(a.routed_blocks + sh.dn_blocks);
#define GLM_PAIR_GU_D(EP, CS, SX)                                                              \
  switch (d / 512) {                                                                           \
    case 2: hipLaunchKernelGGL((select_gate_up_kernel<EP, 2, CS, SX>), g2, dim3(256), lds2, stream, a, sh); break; \
    case 4: hipLaunchKernelGGL((select_gate_up_kernel<EP, 4, CS, SX>), g2, dim3(256), lds2, stream, a, sh); break; \
    case 6: hipLaunchKernelGGL((select_gate_up_kernel<EP, 6, CS, SX>), g2, dim3(256), lds2, stream, a, sh); break; \
    default: hipLaunchKernelGGL((select_gate_up_kernel<EP, 8, CS, SX>), g2, dim3(256), lds2, stream, a, sh); break; \
  }
#define GLM_PAIR_GU(EP, CS)       \
  if (sx) {                       \
    GLM_PAIR_GU_D(EP, CS, true)   \
  } else {                        \
    GLM_PAIR_GU_D(EP, CS, false)  \
  }
#define GLM_PAIR_GU_CS(EP) \
  if (cs == 1) {           \
    GLM_PAIR_GU(EP, 1)     \
  } else {                 \
    GLM_PAIR_GU(EP, 2)     \
  }
  if (epl == 2) {
    GLM_PAIR_GU_CS(2)
  } else if (epl == 4) {
    GLM_PAIR_GU_CS(4)
  } else if (epl == 5) {
    GLM_PAIR_GU_CS(5)
  } else {
    GLM_PAIR_GU_CS(8)
  }
#undef GLM_PAIR_GU_CS
#undef GLM_PAIR_GU
#undef GLM_PAIR_GU_D
  GLM_LAUNCH_CHECK("select_gate_up_kernel");
  return GLM_OK;
}

bool glm_pair_path_supported(int T, int d, int E, int k, int I, int Is) {
  return T >= 1 && T <= kPairMaxT && k <= kPairMaxK && d % 16 == 0 &&
         glm_decode_path_supported(T, d, E, k, I, Is);
}

// The three-kernel token-major layer (T <= 4): logits (+ shared gate/up),
// selection + routed gate/up (+ shared down), down + combine.  The bf16 shared
// expert rides along when sg is given; otherwise shared_ready (bf16 [T][d],
// computed by the caller) or nothing is added.
int glm_pair_path_launch(hipStream_t stream, const uint16_t *x, int T, int d, const float *w,
                         const float *bias, int E, int k, int n_group, int topk_group, int norm,
                         float scale, float *logits, float *weights, uint32_t *indices, int I,
                         const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                         const uint8_t *us, const uint8_t *dw, const uint8_t *ds,
                         const uint16_t *sg, const uint16_t *su, const uint16_t *sd, int Is,
                         float *gp, float *up, uint16_t *hs, float *yp,
                         const uint16_t *shared_ready, uint16_t *h, float limit, float *out,
                         const glm::HcFuse *hc, const uint8_t *sx, long long sx_stride) {
  RouteArgs ra{};
  ra.x = x;
  ra.w = w;
  ra.T = T;
  ra.d = d;
  ra.E = E;
  ra.k = k;
  ra.logits = logits;
  const SharedArgs sh = make_shared_args(x, T, d, sg, su, sd, Is, gp, up, hs, yp, limit);
  int rc = launch_route_logits(stream, ra, sh);
  if (rc) return rc;

  PairArgs a{};
  a.logits = logits;
  a.bias = bias;
  a.T = T;
  a.E = E;
  a.k = k;
  a.n_group = n_group;
  a.topk_group = topk_group;
  a.norm = norm;
  a.scale = scale;
  a.weights = weights;
  a.indices = indices;
  a.x = x;
  a.gw = gw;
  a.gs = gs;
  a.uw = uw;
  a.us = us;
  a.w_stride = (long long)I * (d / 2);
  a.s_stride = (long long)I * (d / 32);
  a.d = d;
  a.I = I;
  a.h = h;
  a.limit = glm_limit_bf16(limit);
  a.tpb = pair_tiles_per_block(T * k, I);
  a.routed_blocks = T * k * (I / 16) / a.tpb;
  a.sx = sx;
  a.sx_stride = sx_stride;
  rc = launch_select_gate_up(stream, a, sh, sg ? glm_decode_shared_cpws(Is) : 1);
  if (rc) return rc;

  PairDownArgs b{};
  b.h = h;
  b.weights = weights;
  b.indices = indices;
  b.dw = dw;
  b.ds = ds;
  b.w_stride = (long long)d * (I / 2);
  b.s_stride = (long long)d * (I / 32);
  b.T = T;
  b.k = k;
  b.I = I;
  b.d = d;
  b.shared = sg ? nullptr : shared_ready;
  b.shared_parts = sg ? yp : nullptr;
  b.nparts = sg ? sh.skd : 0;
  GLM_REQUIRE(b.nparts <= kPairMaxParts, GLM_ERR_UNSUPPORTED_SHAPE,
              "few-token layer: %d shared down partial sums > %d", b.nparts, kPairMaxParts);
  b.out = out;
  if (hc != nullptr) {
    b.hc_res = hc->res;
    b.hc_post = hc->post;
    b.hc_comb = hc->comb;
    b.hc_out = hc->out;
    b.hc = hc->hc;
    b.hc_bf16 = hc->bf16;
  }
  // tiles per block: one while the grid is small; at the real expert
  // geometry (d 4096) two, so the token's h rows and route load once per two tiles
  b.tpb = 1;
  while (b.tpb < 4 && T * (d / 16) / (2 * b.tpb) >= 256 && (d / 16) % (2 * b.tpb) == 0) b.tpb *= 2;
  b.sx = sx;
  b.sx_stride = sx_stride;
  // h rows, then (SX) every wave's decoded down scale rows
  const size_t lds3 = (size_t)k * lds_row_stride(I) * 2 +
                      (sx ? (size_t)k * 16 * b.tpb * (I / 32) : 0);
  const dim3 g3(T * (d / 16) / b.tpb), b3(64 * std::max(k, 4));
#define GLM_PAIR_DN(SX)                                                                      \
  switch (I / 128) {                                                                         \
    case 1: hipLaunchKernelGGL((down_combine_kernel<1, SX>), g3, b3, lds3, stream, b); break; \
    case 2: hipLaunchKernelGGL((down_combine_kernel<2, SX>), g3, b3, lds3, stream, b); break; \
    case 4: hipLaunchKernelGGL((down_combine_kernel<4, SX>), g3, b3, lds3, stream, b); break; \
    case 6: hipLaunchKernelGGL((down_combine_kernel<6, SX>), g3, b3, lds3, stream, b); break; \
    case 8: hipLaunchKernelGGL((down_combine_kernel<8, SX>), g3, b3, lds3, stream, b); break; \
    default: hipLaunchKernelGGL((down_combine_kernel<16, SX>), g3, b3, lds3, stream, b); break; \
  }
  if (sx) {
    GLM_PAIR_DN(true)
  } else {
    GLM_PAIR_DN(false)
  }
#undef GLM_PAIR_DN
  GLM_LAUNCH_CHECK("down_combine_kernel");
  return GLM_OK;
}

int glm_router_validate(const void *x, int T, int d, const void *weight, const void *bias, int E,
                        int k, int n_group, int topk_group, const void *weights,
                        const void *indices);

extern "C" int glm_route_gate_up(void *stream, const float *logits, const float *bias, int T,
                                 int E, int top_k, int n_group, int topk_group, int norm_topk_prob,
                                 float routed_scaling_factor, const uint16_t *x, int d, int I,
                                 const uint8_t *gate_packed, const uint8_t *gate_scales,
                                 const uint8_t *up_packed, const uint8_t *up_scales,
                                 float swiglu_limit, float *weights, uint32_t *indices,
                                 uint16_t *h) {
  glm::clear_error();
  // the router's own checks (logits stand in for its x and weight)
  int rc = glm_router_validate(logits, T, 4, logits, bias, E, top_k, n_group, topk_group, weights,
                               indices);
  if (rc != GLM_OK) return rc;
  GLM_REQUIRE(x && gate_packed && gate_scales && up_packed && up_scales && h,
              GLM_ERR_INVALID_ARGUMENT, "route_gate_up: null pointer argument");
  GLM_REQUIRE(glm_aligned16({x, gate_packed, gate_scales, up_packed, up_scales, h}),
              GLM_ERR_INVALID_ARGUMENT, "route_gate_up: buffers must be 16-byte aligned");
  GLM_REQUIRE(T <= kPairMaxT && top_k <= kPairMaxK && glm_pair_path_supported(T > 0 ? T : 1, d, E, top_k, I, 0),
              GLM_ERR_UNSUPPORTED_SHAPE,
              "route_gate_up: unsupported shape T=%d d=%d E=%d k=%d I=%d (T <= 4, k <= 8, "
              "E <= 448, d/512 in {2,4,6,8}, I/128 in {1,2,4,6,8,16})",
              T, d, E, top_k, I);
  if (T == 0) return GLM_OK;
  PairArgs a{};
  a.logits = logits;
  a.bias = bias;
  a.T = T;
  a.E = E;
  a.k = top_k;
  a.n_group = n_group;
  a.topk_group = topk_group;
  a.norm = norm_topk_prob;
  a.scale = routed_scaling_factor;
  a.weights = weights;
  a.indices = indices;
  a.x = x;
  a.gw = gate_packed;
  a.gs = gate_scales;
  a.uw = up_packed;
  a.us = up_scales;
  a.w_stride = (long long)I * (d / 2);
  a.s_stride = (long long)I * (d / 32);
  a.d = d;
  a.I = I;
  a.h = h;
  a.limit = glm_limit_bf16(swiglu_limit);
  a.tpb = pair_tiles_per_block(T * top_k, I);
  a.routed_blocks = T * top_k * (I / 16) / a.tpb;
  SharedArgs sh{};
  return launch_select_gate_up((hipStream_t)stream, a, sh, 1);
}
