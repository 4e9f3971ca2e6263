// Skinny GEMM ("GEMV" for decode) on MX-quantised or bf16 weights, for gfx950.
//
// out[pos][row] = bf16( sum_k act[arow(pos)][k] * W_e[row][k] )      (NPROJ = 1)
// out[pos][row] = limited_swiglu(bf16(x.Wg_e[row]), bf16(x.Wu_e[row]))  (NPROJ = 2)
//
// Used for the routed expert projections (W_e = expert e of a stacked bank,
// rows grouped by the dispatch offsets), for the shared expert and for the
// resident linears (one "expert", identity activation rows).
//
// Mapping onto CDNA4: a wave owns a 16-row tile of W and a slice of K.  For
// each 128-wide K chunk, lane (r = l & 15, q = l >> 4) reads the 16 bytes of
// packed MXFP4 codes that form ONE complete E8M0 group of row r (group
// 4c + q; a wave's load touches 16 rows x 64 contiguous bytes), converts them
// with v_cvt_scalef32_pk_bf16_fp4 (scale applied in the convert -- the values
// are exact in bf16) and feeds four v_mfma_f32_16x16x32_bf16 whose B operand
// is the activation columns of up to 16 tokens.  The MFMA performs the K
// reduction, so no cross-lane shuffles are needed; the K-split partials of a
// workgroup are reduced through LDS in a fixed wave order, so results are
// deterministic.  K index of MFMA i, slot s of lane (r, q) = c*128 + 32q + 8i + s.
// Routed experts' MXFP4 weights are the bank's (tiled = 1): tile-major, the
// 16-row x 128-K block of tile t and chunk c at byte (t K/128 + c) * 1024
// with lane l's 16 bytes at 16 l, so a wave's load reads 1 KB of contiguous
// memory; resident linears and the shared expert stay row-major.
#include "glm_common.h"

#include <algorithm>

namespace glm {

enum { FMT_BF16 = GLM_FMT_BF16, FMT_MXFP8 = GLM_FMT_MXFP8, FMT_MXFP4 = GLM_FMT_MXFP4 };

struct GemvArgs {
  const uint16_t *act;       // activation rows, bf16 [*][K]
  const int32_t *act_index;  // sorted position -> activation row; nullptr = identity
  const uint8_t *w[2];       // weights of expert 0, per projection
  const uint8_t *s[2];       // scales of expert 0, per projection (unused for bf16)
  long long w_stride;        // bytes between consecutive experts' weights
  long long s_stride;        // bytes between consecutive experts' scales
  int N;                     // rows per expert (output features)
  int K;                     // reduction length
  const int4 *work;          // routed mode: {expert, first row, rows, 0} per slot; nullptr = dense
  int dense_rows;            // dense mode: number of activation rows
  uint16_t *out;             // bf16 [pos][N]
  float limit;               // bf16-rounded swiglu limit (NPROJ == 2)
  int tiled;                 // MXFP4 weights tile-major (the expert bank); N % 16 == K % 128 == 0
};

__host__ __device__ constexpr int row_bytes(int fmt, int K) {
  return fmt == FMT_MXFP4 ? K / 2 : (fmt == FMT_MXFP8 ? K : 2 * K);
}

// Raw bytes of one (16-row x 128-K) chunk for one lane.
template <int FMT>
struct Raw;
template <>
struct Raw<FMT_MXFP4> {
  glm_u32x4 c;
  uint32_t s;
};
template <>
struct Raw<FMT_MXFP8> {
  glm_u32x4 c0, c1;
  uint32_t s;
};
template <>
struct Raw<FMT_BF16> {
  glm_u32x4 v[4];
};

template <int FMT>
__device__ __forceinline__ Raw<FMT> load_raw(const uint8_t *wrow, const uint8_t *srow, int k0,
                                             int q);

template <>
__device__ __forceinline__ Raw<FMT_MXFP4> load_raw<FMT_MXFP4>(const uint8_t *wrow,
                                                              const uint8_t *srow, int k0,
                                                              int q) {
  Raw<FMT_MXFP4> r;
  r.c = *reinterpret_cast<const glm_u32x4 *>(wrow + (k0 >> 1) + 16 * q);
  r.s = srow[(k0 >> 5) + q];
  return r;
}

// The chunk at k0 (a multiple of 128) of a tile-major MXFP4 matrix: wtile
// is this lane's 16-byte piece in its tile's first block.
__device__ __forceinline__ Raw<FMT_MXFP4> load_raw_tiled(const uint8_t *wtile,
                                                         const uint8_t *srow, int k0, int q) {
  Raw<FMT_MXFP4> r;
  r.c = *reinterpret_cast<const glm_u32x4 *>(wtile + (size_t)(k0 >> 7) * 1024);
  r.s = srow[(k0 >> 5) + q];
  return r;
}

template <>
__device__ __forceinline__ Raw<FMT_MXFP8> load_raw<FMT_MXFP8>(const uint8_t *wrow,
                                                              const uint8_t *srow, int k0,
                                                              int q) {
  Raw<FMT_MXFP8> r;
  const glm_u32x4 *p = reinterpret_cast<const glm_u32x4 *>(wrow + k0 + 32 * q);
  r.c0 = p[0];
  r.c1 = p[1];
  r.s = srow[(k0 >> 5) + q];
  return r;
}

template <>
__device__ __forceinline__ Raw<FMT_BF16> load_raw<FMT_BF16>(const uint8_t *wrow,
                                                            const uint8_t *srow, int k0, int q) {
  Raw<FMT_BF16> r;
  const glm_u32x4 *p = reinterpret_cast<const glm_u32x4 *>(wrow + 2 * (k0 + 32 * q));
#pragma unroll
  for (int i = 0; i < 4; ++i) r.v[i] = p[i];
  return r;
}

// Dequantise one raw chunk into the four MFMA A fragments.
template <int FMT>
__device__ __forceinline__ void to_frags(const Raw<FMT> &r, glm_bf16x8 a[4]);

template <>
__device__ __forceinline__ void to_frags<FMT_MXFP4>(const Raw<FMT_MXFP4> &r, glm_bf16x8 a[4]) {
  const float sc = e8m0_to_f32(r.s);
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = mxfp4_word_to_bf16x8(r.c[i], sc);
}

template <>
__device__ __forceinline__ void to_frags<FMT_MXFP8>(const Raw<FMT_MXFP8> &r, glm_bf16x8 a[4]) {
  const float sc = e8m0_to_f32(r.s);
  a[0] = mxfp8_words_to_bf16x8(r.c0[0], r.c0[1], sc);
  a[1] = mxfp8_words_to_bf16x8(r.c0[2], r.c0[3], sc);
  a[2] = mxfp8_words_to_bf16x8(r.c1[0], r.c1[1], sc);
  a[3] = mxfp8_words_to_bf16x8(r.c1[2], r.c1[3], sc);
}

template <>
__device__ __forceinline__ void to_frags<FMT_BF16>(const Raw<FMT_BF16> &r, glm_bf16x8 a[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = __builtin_bit_cast(glm_bf16x8, r.v[i]);
}

constexpr int kMaxTiles = 4;  // token tiles of 16 held in registers per pass

template <int FMT, int NPROJ, int CPW, bool TILED>
__global__ __launch_bounds__(512) void mx_gemv_kernel(const GemvArgs args) {
  static_assert(!TILED || FMT == FMT_MXFP4, "tile-major weights are MXFP4");
  extern __shared__ glm_f32x4 red[];  // [ksplit][kMaxTiles][NPROJ][64]
  const int ksplit = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int q = lane >> 4;

  int e = 0, base = 0, n = args.dense_rows;
  if (args.work != nullptr) {
    const int4 wk = args.work[blockIdx.y];
    if (wk.x < 0) return;
    e = wk.x;
    base = wk.y;
    n = wk.z;
  }
  if (n <= 0) return;
  const int K = args.K;
  const int N = args.N;
  const int row0 = blockIdx.x * 16;
  const int rb = row_bytes(FMT, K);
  const uint8_t *wrow[NPROJ];
  const uint8_t *srow[NPROJ];
#pragma unroll
  for (int p = 0; p < NPROJ; ++p) {
    wrow[p] = args.w[p] + (long long)e * args.w_stride +
              (TILED ? (long long)row0 * rb + 16 * lane : (long long)(row0 + r) * rb);
    srow[p] = FMT == FMT_BF16 ? nullptr
                              : args.s[p] + (long long)e * args.s_stride +
                                    (long long)(row0 + r) * (K >> 5);
  }
  const int kbase = wave * CPW * 128;

  for (int p0 = 0; p0 < n; p0 += 16 * kMaxTiles) {
    const int ntiles = min(kMaxTiles, (n - p0 + 15) >> 4);
    // Activation row of this lane's token column, per tile.  Columns past the
    // last row read a valid row (the last one) instead of branching: an MFMA
    // output column depends only on its own B column, and those columns are
    // never stored.  Branch-free loads let every load below be in flight at
    // once.
    int arow[kMaxTiles];
#pragma unroll
    for (int tt = 0; tt < kMaxTiles; ++tt) {
      const int pair = min(p0 + tt * 16 + r, n - 1);
      arow[tt] = args.act_index ? args.act_index[base + pair] : base + pair;
    }
    // Issue every weight load of this wave, then tile 0's activation
    // fragments for all chunks, before the first wait.
    Raw<FMT> raw[NPROJ][CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int p = 0; p < NPROJ; ++p) {
        if constexpr (TILED)
          raw[p][c] = load_raw_tiled(wrow[p], srow[p], kbase + c * 128, q);
        else
          raw[p][c] = load_raw<FMT>(wrow[p], srow[p], kbase + c * 128, q);
      }
    glm_bf16x8 b0[CPW][4];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const glm_bf16x8 *src = reinterpret_cast<const glm_bf16x8 *>(
          args.act + (long long)arow[0] * K + kbase + c * 128 + 32 * q);
#pragma unroll
      for (int i = 0; i < 4; ++i) b0[c][i] = src[i];
    }

    glm_f32x4 acc[kMaxTiles][NPROJ];
#pragma unroll
    for (int tt = 0; tt < kMaxTiles; ++tt)
#pragma unroll
      for (int p = 0; p < NPROJ; ++p) acc[tt][p] = glm_f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      glm_bf16x8 a[NPROJ][4];
#pragma unroll
      for (int p = 0; p < NPROJ; ++p) to_frags<FMT>(raw[p][c], a[p]);
      const int k0 = kbase + c * 128 + 32 * q;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int p = 0; p < NPROJ; ++p)
          acc[0][p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[p][i], b0[c][i], acc[0][p], 0, 0, 0);
#pragma unroll
      for (int tt = 1; tt < kMaxTiles; ++tt) {
        if (tt < ntiles) {
          const glm_bf16x8 *src =
              reinterpret_cast<const glm_bf16x8 *>(args.act + (long long)arow[tt] * K + k0);
          glm_bf16x8 b[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) b[i] = src[i];
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int p = 0; p < NPROJ; ++p)
              acc[tt][p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[p][i], b[i], acc[tt][p], 0, 0, 0);
        }
      }
    }

    // Fixed-order reduction of the K-split partials.
    if (ksplit > 1) {
#pragma unroll
      for (int tt = 0; tt < kMaxTiles; ++tt)
        if (tt < ntiles)
#pragma unroll
          for (int p = 0; p < NPROJ; ++p)
            red[((wave * kMaxTiles + tt) * NPROJ + p) * 64 + lane] = acc[tt][p];
      __syncthreads();
    }
    // Wave w finishes tiles tt = w, w + ksplit, ...
    for (int tt = (ksplit > 1 ? wave : 0); tt < ntiles; tt += ksplit) {
      glm_f32x4 sum[NPROJ];
      if (ksplit > 1) {
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) {
          sum[p] = red[((0 * kMaxTiles + tt) * NPROJ + p) * 64 + lane];
          for (int w = 1; w < ksplit; ++w) sum[p] += red[((w * kMaxTiles + tt) * NPROJ + p) * 64 + lane];
        }
      } else {
        // ksplit == 1: the loop visits every tile; select it from registers.
#pragma unroll
        for (int t2 = 0; t2 < kMaxTiles; ++t2)
          if (t2 == tt)
#pragma unroll
            for (int p = 0; p < NPROJ; ++p) sum[p] = acc[t2][p];
      }
      // Lane (r, q) holds rows 4q..4q+3 of the tile for token column r.
      const int pair = p0 + tt * 16 + r;
      if (pair < n) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          if (NPROJ == 2) {
            const float g = bf16_round(sum[0][m]);
            const float u = bf16_round(sum[NPROJ - 1][m]);
            o[m] = f32_to_bf16(limited_swiglu(g, u, args.limit));
          } else {
            o[m] = f32_to_bf16(sum[0][m]);
          }
        }
        uint2 packed;
        packed.x = o[0] | (o[1] << 16);
        packed.y = o[2] | (o[3] << 16);
        *reinterpret_cast<uint2 *>(args.out + (long long)(base + pair) * N + row0 + 4 * q) = packed;
      }
    }
    if (ksplit > 1) __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Few-token linear on the vector ALUs (T <= 4).  With one to four token rows
// an MFMA tile computes 16 columns for each one kept, and its 16-row tiles
// would leave half of the CUs idle at N = 2048, so each wave owns two output
// rows here and a block of four waves eight: lane l takes the 32-wide K
// slices l, l + 64, ... of both rows (one 32-byte load per row for MXFP8),
// converts them to bf16 (exact) and forms packed bf16 dot products with each
// token's slice; the 64 lane partials are added in a fixed butterfly order.
// XF32: x is f32 and every value is rounded to bf16 (RNE) as it is read.
// ---------------------------------------------------------------------------
constexpr int kRowsPerWave = 2;
constexpr int kLinearMaxT = 4;

struct LinearRowsArgs {
  const void *x;
  int T, K, N;
  const uint8_t *w, *s;
  uint16_t *y;
  // linear_mx8_kernel<true, true>: RMSNorm of the f32 rows first (weight f32
  // [K] or nullptr)
  const float *norm_w;
  float eps;
};

__device__ __forceinline__ glm_bf16x2 bf16_pair(const glm_bf16x8 &v, int p) {
  glm_bf16x2 r;
  r[0] = v[2 * p];
  r[1] = v[2 * p + 1];
  return r;
}

__device__ __forceinline__ glm_u32x4 nt_load16(const uint8_t *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const glm_u32x4 *>(p));
}

// One lane's 32-wide K slice of one weight row, as loaded.
template <int FMT>
struct RowSlice {
  glm_u32x4 c[FMT == FMT_MXFP8 ? 2 : (FMT == FMT_MXFP4 ? 1 : 4)];
  uint32_t s;
};

template <int FMT>
__device__ __forceinline__ RowSlice<FMT> load_slice(const uint8_t *wrow, const uint8_t *srow, int sl) {
  RowSlice<FMT> r;
  constexpr int n = FMT == FMT_MXFP8 ? 2 : (FMT == FMT_MXFP4 ? 1 : 4);
#pragma unroll
  for (int i = 0; i < n; ++i) r.c[i] = nt_load16(wrow + (size_t)sl * 16 * n + 16 * i);
  r.s = FMT == FMT_BF16 ? 0u : srow[sl];
  return r;
}

template <int FMT>
__device__ __forceinline__ void slice_bf16(const RowSlice<FMT> &r, glm_bf16x8 out[4]) {
  if constexpr (FMT == FMT_MXFP8) {
    const float sc = e8m0_to_f32(r.s);
    out[0] = mxfp8_words_to_bf16x8(r.c[0][0], r.c[0][1], sc);
    out[1] = mxfp8_words_to_bf16x8(r.c[0][2], r.c[0][3], sc);
    out[2] = mxfp8_words_to_bf16x8(r.c[1][0], r.c[1][1], sc);
    out[3] = mxfp8_words_to_bf16x8(r.c[1][2], r.c[1][3], sc);
  } else if constexpr (FMT == FMT_MXFP4) {
    const float sc = e8m0_to_f32(r.s);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = mxfp4_word_to_bf16x8(r.c[0][i], sc);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __builtin_bit_cast(glm_bf16x8, r.c[i]);
  }
}

template <bool XF32>
__device__ __forceinline__ void slice_act(const void *x, size_t off, glm_bf16x8 out[4]) {
  if constexpr (XF32) {
    const glm_f32x4 *p = reinterpret_cast<const glm_f32x4 *>(static_cast<const float *>(x) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const glm_f32x4 a = p[2 * i], b = p[2 * i + 1];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        out[i][m] = (__bf16)a[m];
        out[i][4 + m] = (__bf16)b[m];
      }
    }
  } else {
    const glm_bf16x8 *p = reinterpret_cast<const glm_bf16x8 *>(static_cast<const uint16_t *>(x) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = p[i];
  }
}

template <int FMT, bool XF32>
__global__ __launch_bounds__(256) void linear_rows_kernel(const LinearRowsArgs a) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kRowsPerWave;
  const int K = a.K, rb = row_bytes(FMT, K);
  float acc[kRowsPerWave][kLinearMaxT];
#pragma unroll
  for (int rr = 0; rr < kRowsPerWave; ++rr)
#pragma unroll
    for (int t = 0; t < kLinearMaxT; ++t) acc[rr][t] = 0.0f;
  for (int sl = lane; sl < K / 32; sl += 64) {
    // the weight slices and token 0's slice go out together, before any wait
    RowSlice<FMT> raw[kRowsPerWave];
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr)
      raw[rr] = load_slice<FMT>(a.w + (size_t)(row0 + rr) * rb,
                                FMT == FMT_BF16 ? nullptr : a.s + (size_t)(row0 + rr) * (K / 32), sl);
    glm_bf16x8 xv[4];
    slice_act<XF32>(a.x, (size_t)sl * 32, xv);
    __builtin_amdgcn_sched_barrier(0);
    glm_bf16x8 wv[kRowsPerWave][4];
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) slice_bf16<FMT>(raw[rr], wv[rr]);
#pragma unroll
    for (int t = 0; t < kLinearMaxT; ++t) {
      if (t < a.T) {
        if (t > 0) slice_act<XF32>(a.x, (size_t)t * K + sl * 32, xv);
#pragma unroll
        for (int rr = 0; rr < kRowsPerWave; ++rr)
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int p = 0; p < 4; ++p)
              acc[rr][t] = __builtin_amdgcn_fdot2_f32_bf16(bf16_pair(wv[rr][i], p),
                                                           bf16_pair(xv[i], p), acc[rr][t], false);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kLinearMaxT; ++t) {
    if (t < a.T) {
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const float v = wave_sum(acc[rr][t]);
        if (lane == 0) a.y[(size_t)t * a.N + row0 + rr] = (uint16_t)f32_to_bf16(v);
      }
    }
  }
}

// MXFP8 weights with the K columns interleaved over the lanes: in step j
// lane l takes columns 256 j + 4 l .. + 3 of its wave's two rows (one dword
// of codes and its scale byte per row) and of each token (16 bytes of f32 or
// 8 of bf16 x).  Every load instruction of the wave then reads one contiguous
// stretch (256 B of codes, 1 KB of f32 x); with 32-wide slices per lane each
// 16-byte piece of a lane's x lies on its own 128-byte line, 64 lines per
// instruction.  The same kernel serves bf16 and f32 x, so the two entry
// points agree bit for bit.
constexpr int kMx8Steps = 8;  // 256-column steps per pass (K = 2048: one pass)

template <bool XF32>
__device__ __forceinline__ void x_cols4(const void *x, size_t off, glm_bf16x2 &p0, glm_bf16x2 &p1) {
  if constexpr (XF32) {
    const glm_f32x4 v = *reinterpret_cast<const glm_f32x4 *>(static_cast<const float *>(x) + off);
    p0[0] = (__bf16)v[0];
    p0[1] = (__bf16)v[1];
    p1[0] = (__bf16)v[2];
    p1[1] = (__bf16)v[3];
  } else {
    typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
    const bf16x4 v = *reinterpret_cast<const bf16x4 *>(static_cast<const uint16_t *>(x) + off);
    p0 = __builtin_shufflevector(v, v, 0, 1);
    p1 = __builtin_shufflevector(v, v, 2, 3);
  }
}

// NORM (f32 x only): every x row is replaced by its RMSNorm, x * (1 /
// sqrt(mean(x^2) + eps)) * w (the product rounded after each factor, as
// rms_norm_kernel), before the rounding to bf16.  The wave's loads of a pass
// cover the whole row when K <= 256 kMx8Steps, so the sum of squares comes
// from them; longer rows take one pre-pass over the row.
template <bool XF32, bool NORM = false>
__global__ __launch_bounds__(256) void linear_mx8_kernel(const LinearRowsArgs a) {
  static_assert(XF32 || !NORM, "the fused RMSNorm reads f32 rows");
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kRowsPerWave;
  const int K = a.K, steps = K / 256;
  float acc[kRowsPerWave][kLinearMaxT];
#pragma unroll
  for (int rr = 0; rr < kRowsPerWave; ++rr)
#pragma unroll
    for (int t = 0; t < kLinearMaxT; ++t) acc[rr][t] = 0.0f;
  const bool one_pass = steps <= kMx8Steps;
  float inv[kLinearMaxT];
  auto norm_inv = [&](float ss) {
    return 1.0f / sqrtf(wave_sum(ss) / (float)K + a.eps);
  };
  if constexpr (NORM) {
    if (!one_pass) {
#pragma unroll
      for (int t = 0; t < kLinearMaxT; ++t) {
        float ss = 0.0f;
        if (t < a.T) {
          for (int c = 4 * lane; c < K; c += 256) {
            const glm_f32x4 v = *reinterpret_cast<const glm_f32x4 *>(
                static_cast<const float *>(a.x) + (size_t)t * K + c);
            ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
          }
          inv[t] = norm_inv(ss);
        }
      }
    }
  }
  for (int j0 = 0; j0 < steps; j0 += kMx8Steps) {
    // every load of the pass goes out before any use (steps past the end
    // repeat the last one and are not added)
    uint32_t code[kMx8Steps][kRowsPerWave], sb[kMx8Steps][kRowsPerWave];
    glm_bf16x2 xp[kMx8Steps][2];
#pragma unroll
    for (int jj = 0; jj < kMx8Steps; ++jj) {
      const int col = 256 * min(j0 + jj, steps - 1) + 4 * lane;
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        code[jj][rr] = __builtin_nontemporal_load(
            reinterpret_cast<const uint32_t *>(a.w + (size_t)(row0 + rr) * K + col));
        sb[jj][rr] = a.s[(size_t)(row0 + rr) * (K / 32) + col / 32];
      }
    }
    glm_f32x4 xf[kMx8Steps], nw[kMx8Steps];
    if constexpr (NORM) {
#pragma unroll
      for (int jj = 0; jj < kMx8Steps; ++jj) {
        const int col = 256 * min(j0 + jj, steps - 1) + 4 * lane;
        xf[jj] = *reinterpret_cast<const glm_f32x4 *>(static_cast<const float *>(a.x) + col);
        nw[jj] = a.norm_w != nullptr ? *reinterpret_cast<const glm_f32x4 *>(a.norm_w + col)
                                     : glm_f32x4{1.f, 1.f, 1.f, 1.f};
      }
    } else {
#pragma unroll
      for (int jj = 0; jj < kMx8Steps; ++jj)
        x_cols4<XF32>(a.x, 256 * min(j0 + jj, steps - 1) + 4 * lane, xp[jj][0], xp[jj][1]);
    }
    // token t's normalised columns of this pass as bf16 pairs (the sum of
    // squares from the pass's own values when it covers the row; steps past
    // the end repeat the last one and are left out of it)
    auto norm_cols = [&](int t) {
      if constexpr (NORM) {
        if (one_pass) {
          float ss = 0.0f;
#pragma unroll
          for (int jj = 0; jj < kMx8Steps; ++jj)
            if (j0 + jj < steps)
              ss += xf[jj][0] * xf[jj][0] + xf[jj][1] * xf[jj][1] + xf[jj][2] * xf[jj][2] +
                    xf[jj][3] * xf[jj][3];
          inv[t] = norm_inv(ss);
        }
#pragma unroll
        for (int jj = 0; jj < kMx8Steps; ++jj) {
          float v[4];
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            v[m] = xf[jj][m] * inv[t];
            if (a.norm_w != nullptr) v[m] *= nw[jj][m];
          }
          xp[jj][0][0] = (__bf16)v[0];
          xp[jj][0][1] = (__bf16)v[1];
          xp[jj][1][0] = (__bf16)v[2];
          xp[jj][1][1] = (__bf16)v[3];
        }
      }
    };
    __builtin_amdgcn_sched_barrier(0);
    glm_bf16x2 wp[kMx8Steps][kRowsPerWave][2];
#pragma unroll
    for (int jj = 0; jj < kMx8Steps; ++jj)
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const float sc = e8m0_to_f32(sb[jj][rr]);
        wp[jj][rr][0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(code[jj][rr], sc, false);
        wp[jj][rr][1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(code[jj][rr], sc, true);
      }
#pragma unroll
    for (int t = 0; t < kLinearMaxT; ++t) {
      if (t < a.T) {
        if (t > 0) {
#pragma unroll
          for (int jj = 0; jj < kMx8Steps; ++jj) {
            const size_t off = (size_t)t * K + 256 * min(j0 + jj, steps - 1) + 4 * lane;
            if constexpr (NORM)
              xf[jj] = *reinterpret_cast<const glm_f32x4 *>(static_cast<const float *>(a.x) + off);
            else
              x_cols4<XF32>(a.x, off, xp[jj][0], xp[jj][1]);
          }
        }
        norm_cols(t);
#pragma unroll
        for (int jj = 0; jj < kMx8Steps; ++jj) {
          if (j0 + jj < steps) {
#pragma unroll
            for (int rr = 0; rr < kRowsPerWave; ++rr) {
              acc[rr][t] = __builtin_amdgcn_fdot2_f32_bf16(wp[jj][rr][0], xp[jj][0], acc[rr][t], false);
              acc[rr][t] = __builtin_amdgcn_fdot2_f32_bf16(wp[jj][rr][1], xp[jj][1], acc[rr][t], false);
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kLinearMaxT; ++t) {
    if (t < a.T) {
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const float v = wave_sum(acc[rr][t]);
        if (lane == 0) a.y[(size_t)t * a.N + row0 + rr] = (uint16_t)f32_to_bf16(v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Generic fallback for shapes the MFMA tiling does not cover (K % 128 or
// N % 16 non-zero; e.g. the tiny test geometries).  One thread per output.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float e2m1_value(uint32_t code) {
  const float mags[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float m = mags[code & 7];
  return (code & 8) ? -m : m;
}

__device__ __forceinline__ float e4m3fn_value(uint32_t byte) {
  const uint32_t e = (byte >> 3) & 15, m = byte & 7;
  float v;
  if (e == 0) v = ldexpf((float)m / 8.0f, -6);
  else if (e == 15 && m == 7) v = __uint_as_float(0x7fc00000u);
  else v = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
  return (byte & 0x80) ? -v : v;
}

template <int FMT>
__device__ __forceinline__ float weight_at(const uint8_t *wrow, const uint8_t *srow, int k) {
  if (FMT == FMT_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t *>(wrow)[k]);
  const float sc = e8m0_to_f32(srow[k >> 5]);
  if (FMT == FMT_MXFP4) {
    const uint32_t byte = wrow[k >> 1];
    return e2m1_value((k & 1) ? (byte >> 4) : (byte & 15)) * sc;
  }
  return e4m3fn_value(wrow[k]) * sc;
}

template <int FMT, int NPROJ>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const GemvArgs args) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  int e = 0, base = 0, n = args.dense_rows;
  if (args.work != nullptr) {
    const int4 wk = args.work[blockIdx.y];
    if (wk.x < 0) return;
    e = wk.x;
    base = wk.y;
    n = wk.z;
  }
  if (row >= args.N) return;
  const int K = args.K;
  const int rb = row_bytes(FMT, K);
  // tile-major MXFP4 (the bank's layout of a geometry the MFMA path has no
  // K split for): element k of the row sits in piece mxfp4_tile_piece of the
  // matrix
  const bool tiled = FMT == FMT_MXFP4 && args.tiled;
  const uint8_t *wmat[NPROJ];
  const uint8_t *srow[NPROJ];
  for (int p = 0; p < NPROJ; ++p) {
    wmat[p] = args.w[p] + (long long)e * args.w_stride;
    srow[p] = FMT == FMT_BF16 ? nullptr
                              : args.s[p] + (long long)e * args.s_stride + (long long)row * (K >> 5);
  }
  for (int pair = 0; pair < n; ++pair) {
    const int arow = args.act_index ? args.act_index[base + pair] : base + pair;
    const uint16_t *xr = args.act + (long long)arow * K;
    float acc[NPROJ];
    for (int p = 0; p < NPROJ; ++p) {
      float a = 0.0f;
      if (tiled) {
        for (int k = 0; k < K; ++k) {
          const uint8_t *piece = wmat[p] + 16 * mxfp4_tile_piece(row, k >> 5, K);
          const uint32_t byte = piece[(k >> 1) & 15];
          const float wk = e2m1_value((k & 1) ? (byte >> 4) : (byte & 15)) * e8m0_to_f32(srow[p][k >> 5]);
          a = fmaf(bf16_to_f32(xr[k]), wk, a);
        }
      } else {
        const uint8_t *wrow = wmat[p] + (long long)row * rb;
        for (int k = 0; k < K; ++k) a = fmaf(bf16_to_f32(xr[k]), weight_at<FMT>(wrow, srow[p], k), a);
      }
      acc[p] = a;
    }
    float v;
    if (NPROJ == 2) v = limited_swiglu(bf16_round(acc[0]), bf16_round(acc[NPROJ - 1]), args.limit);
    else v = acc[0];
    args.out[(long long)(base + pair) * args.N + row] = (uint16_t)f32_to_bf16(v);
  }
}

}  // namespace glm

using glm::GemvArgs;

extern "C" int glm_mxfp4_is_tiled(int rows, int K);

// Picks the K split for the MFMA path: total chunks KC = K/128 = ksplit*cpw.
static bool choose_split(int fmt, int nproj, int K, int *ksplit, int *cpw) {
  if (K % 128 != 0) return false;
  const int kc = K / 128;
  // bf16 gate/up holds two projections of bf16 rows: 2 chunks per wave keep
  // it at 3 waves per SIMD; 4 chunks (244 registers, 2 waves per SIMD) only
  // when no split with 2 fits (K = 4096 and beyond)
  const bool bf16_pair = fmt == GLM_FMT_BF16 && nproj == 2;
  for (int max_cpw : {bf16_pair ? 2 : 4, 4}) {
    // Prefer a 4-wave split, then 2, 8, 1; within that the largest cpw that fits.
    const int splits[] = {4, 2, 8, 1, 3, 6};
    for (int s : splits) {
      if (kc % s) continue;
      const int c = kc / s;
      if (c >= 1 && c <= max_cpw) {
        *ksplit = s;
        *cpw = c;
        return true;
      }
    }
  }
  return false;
}

template <int FMT, int NPROJ, bool TILED>
static void launch_mfma(hipStream_t stream, const GemvArgs &a, int grid_y, int ksplit, int cpw) {
  dim3 grid(a.N / 16, grid_y);
  dim3 block(64 * ksplit);
  const size_t lds = ksplit > 1 ? (size_t)ksplit * glm::kMaxTiles * NPROJ * 64 * 16 : 0;
  switch (cpw) {
    case 1:
      hipLaunchKernelGGL((glm::mx_gemv_kernel<FMT, NPROJ, 1, TILED>), grid, block, lds, stream, a);
      break;
    case 2:
      hipLaunchKernelGGL((glm::mx_gemv_kernel<FMT, NPROJ, 2, TILED>), grid, block, lds, stream, a);
      break;
    case 3:
      hipLaunchKernelGGL((glm::mx_gemv_kernel<FMT, NPROJ, 3, TILED>), grid, block, lds, stream, a);
      break;
    default:
      hipLaunchKernelGGL((glm::mx_gemv_kernel<FMT, NPROJ, 4, TILED>), grid, block, lds, stream, a);
      break;
  }
}

template <int FMT, int NPROJ>
static int launch_fmt(hipStream_t stream, const GemvArgs &a, int grid_y) {
  int ksplit = 0, cpw = 0;
  const bool mfma = a.N % 16 == 0 && choose_split(FMT, NPROJ, a.K, &ksplit, &cpw);
  GLM_REQUIRE(!a.tiled || (FMT == GLM_FMT_MXFP4 && glm::mxfp4_tiled(a.N, a.K)),
              GLM_ERR_UNSUPPORTED_SHAPE,
              "gemv: tile-major weights need MXFP4, N %% 16 == 0 and K %% 128 == 0 (N=%d K=%d)",
              a.N, a.K);
  if (mfma) {
    if constexpr (FMT == GLM_FMT_MXFP4) {
      if (a.tiled) launch_mfma<FMT, NPROJ, true>(stream, a, grid_y, ksplit, cpw);
      else launch_mfma<FMT, NPROJ, false>(stream, a, grid_y, ksplit, cpw);
    } else {
      launch_mfma<FMT, NPROJ, false>(stream, a, grid_y, ksplit, cpw);
    }
    GLM_LAUNCH_CHECK("mx_gemv_kernel");
    return GLM_OK;
  }
  dim3 grid((a.N + 255) / 256, grid_y);
  hipLaunchKernelGGL((glm::gemv_generic_kernel<FMT, NPROJ>), grid, dim3(256), 0, stream, a);
  GLM_LAUNCH_CHECK("gemv_generic_kernel");
  return GLM_OK;
}

// grid_y = number of expert slots to cover (routed) or 1 (dense).
int glm_gemv_launch(hipStream_t stream, int fmt, int nproj, const GemvArgs &a, int grid_y) {
  if (grid_y <= 0) return GLM_OK;
  if (nproj == 2) {
    switch (fmt) {
      case GLM_FMT_MXFP4: return launch_fmt<GLM_FMT_MXFP4, 2>(stream, a, grid_y);
      case GLM_FMT_MXFP8: return launch_fmt<GLM_FMT_MXFP8, 2>(stream, a, grid_y);
      default: return launch_fmt<GLM_FMT_BF16, 2>(stream, a, grid_y);
    }
  }
  switch (fmt) {
    case GLM_FMT_MXFP4: return launch_fmt<GLM_FMT_MXFP4, 1>(stream, a, grid_y);
    case GLM_FMT_MXFP8: return launch_fmt<GLM_FMT_MXFP8, 1>(stream, a, grid_y);
    default: return launch_fmt<GLM_FMT_BF16, 1>(stream, a, grid_y);
  }
}

static int check_fmt(int fmt) {
  GLM_REQUIRE(fmt == GLM_FMT_BF16 || fmt == GLM_FMT_MXFP8 || fmt == GLM_FMT_MXFP4,
              GLM_ERR_INVALID_ARGUMENT, "unknown weight format %d", fmt);
  return GLM_OK;
}

int glm_decode_gate_up_launch(hipStream_t stream, const uint16_t *x, int T, int d, int I, int E,
                              int k, const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                              const uint8_t *us, const int32_t *pair_token, const int4 *work,
                              uint16_t *h, float limit, const uint16_t *sg, const uint16_t *su,
                              int Is, uint16_t *hs);
int glm_decode_down_launch(hipStream_t stream, const uint16_t *h, int T, int k, int I, int d,
                           int E, const uint8_t *dw, const uint8_t *ds, const int4 *work,
                           uint16_t *y, const uint16_t *sd, int Is, uint16_t *hs, float *yp);
bool glm_decode_gate_up_supported(int d, int I);
bool glm_decode_down_supported(int I, int d);

int glm_gate_up_launch(hipStream_t stream, const uint16_t *x, int T, int d, int I, int E, int k,
                       const uint8_t *gw, const uint8_t *gs, const uint8_t *uw, const uint8_t *us,
                       const int32_t *pair_token, const int4 *work, float limit, uint16_t *h) {
  if (glm_decode_gate_up_supported(d, I))
    return glm_decode_gate_up_launch(stream, x, T, d, I, E, k, gw, gs, uw, us, pair_token, work,
                                     h, limit, nullptr, nullptr, 0, nullptr);
  GemvArgs a{};
  a.act = x;
  a.act_index = pair_token;
  a.w[0] = gw;
  a.w[1] = uw;
  a.s[0] = gs;
  a.s[1] = us;
  a.w_stride = (long long)I * (d / 2);
  a.s_stride = (long long)I * (d / 32);
  a.N = I;
  a.K = d;
  a.work = work;
  a.out = h;
  a.limit = glm_limit_bf16(limit);
  a.tiled = glm_mxfp4_is_tiled(I, d);  // the bank's layout of this geometry
  const int slots = std::min(E, T * k);
  return glm_gemv_launch(stream, GLM_FMT_MXFP4, 2, a, slots);
}

int glm_down_launch(hipStream_t stream, const uint16_t *h, int T, int k, int I, int d, int E,
                    const uint8_t *dw, const uint8_t *ds, const int4 *work, uint16_t *y) {
  if (glm_decode_down_supported(I, d))
    return glm_decode_down_launch(stream, h, T, k, I, d, E, dw, ds, work, y, nullptr, 0, nullptr,
                                  nullptr);
  GemvArgs a{};
  a.act = h;
  a.act_index = nullptr;
  a.w[0] = a.w[1] = dw;
  a.s[0] = a.s[1] = ds;
  a.w_stride = (long long)d * (I / 2);
  a.s_stride = (long long)d * (I / 32);
  a.N = d;
  a.K = I;
  a.work = work;
  a.out = y;
  a.tiled = glm_mxfp4_is_tiled(d, I);
  const int slots = std::min(E, T * k);
  return glm_gemv_launch(stream, GLM_FMT_MXFP4, 1, a, slots);
}

// Whether the few-token vector-ALU linear covers this call.
static bool linear_rows_supported(int T, int in_dims, int out_dims) {
  return T >= 1 && T <= glm::kLinearMaxT && in_dims % 32 == 0 &&
         out_dims % (4 * glm::kRowsPerWave) == 0;
}

template <bool XF32>
static int launch_linear_rows(hipStream_t stream, const void *x, int T, int in_dims,
                              const void *weight, const uint8_t *scales, int fmt, int out_dims,
                              uint16_t *y) {
  const glm::LinearRowsArgs a{x, T, in_dims, out_dims, static_cast<const uint8_t *>(weight), scales,
                              y, nullptr, 0.0f};
  const dim3 grid(out_dims / (4 * glm::kRowsPerWave)), block(256);
  switch (fmt) {
    case GLM_FMT_MXFP4: hipLaunchKernelGGL((glm::linear_rows_kernel<GLM_FMT_MXFP4, XF32>), grid, block, 0, stream, a); break;
    case GLM_FMT_MXFP8:
      if (in_dims % 256 == 0)
        hipLaunchKernelGGL((glm::linear_mx8_kernel<XF32>), grid, block, 0, stream, a);
      else
        hipLaunchKernelGGL((glm::linear_rows_kernel<GLM_FMT_MXFP8, XF32>), grid, block, 0, stream, a);
      break;
    default: hipLaunchKernelGGL((glm::linear_rows_kernel<GLM_FMT_BF16, XF32>), grid, block, 0, stream, a); break;
  }
  GLM_LAUNCH_CHECK("linear_rows_kernel");
  return GLM_OK;
}

int glm_linear_launch(hipStream_t stream, const uint16_t *x, int T, int in_dims,
                      const void *weight, const uint8_t *scales, int fmt, int out_dims,
                      uint16_t *y) {
  if (linear_rows_supported(T, in_dims, out_dims))
    return launch_linear_rows<false>(stream, x, T, in_dims, weight, scales, fmt, out_dims, y);
  GemvArgs a{};
  a.act = x;
  a.w[0] = a.w[1] = static_cast<const uint8_t *>(weight);
  a.s[0] = a.s[1] = scales;
  a.N = out_dims;
  a.K = in_dims;
  a.dense_rows = T;
  a.out = y;
  return glm_gemv_launch(stream, fmt, 1, a, T > 0 ? 1 : 0);
}

bool glm_grouped_dense_mlp_supported(int T, int d, int I, int fmt);
int glm_grouped_dense_mlp_launch(hipStream_t stream, const uint16_t *x, int T, int d, int I,
                                 const uint16_t *gw, const uint16_t *uw, const uint16_t *dw,
                                 float limit, uint16_t *h, uint16_t *out);

int glm_mlp_launch(hipStream_t stream, const uint16_t *x, int T, int d, int I, int fmt,
                   const void *gw, const uint8_t *gs, const void *uw, const uint8_t *us,
                   const void *dw, const uint8_t *ds, float limit, uint16_t *h, uint16_t *out) {
  if (glm_grouped_dense_mlp_supported(T, d, I, fmt))  // many tokens: tiled MFMA GEMMs
    return glm_grouped_dense_mlp_launch(stream, x, T, d, I, static_cast<const uint16_t *>(gw),
                                        static_cast<const uint16_t *>(uw),
                                        static_cast<const uint16_t *>(dw), limit, h, out);
  GemvArgs a{};
  a.act = x;
  a.w[0] = static_cast<const uint8_t *>(gw);
  a.w[1] = static_cast<const uint8_t *>(uw);
  a.s[0] = gs;
  a.s[1] = us;
  a.N = I;
  a.K = d;
  a.dense_rows = T;
  a.out = h;
  a.limit = glm_limit_bf16(limit);
  int rc = glm_gemv_launch(stream, fmt, 2, a, T > 0 ? 1 : 0);
  if (rc != GLM_OK) return rc;
  return glm_linear_launch(stream, h, T, I, dw, ds, fmt, d, out);
}

static int check_mx_geometry(const char *who, int fmt, int in_dims, int out_dims) {
  GLM_REQUIRE(in_dims > 0 && out_dims > 0, GLM_ERR_INVALID_ARGUMENT, "%s: invalid dims %d x %d",
              who, out_dims, in_dims);
  GLM_REQUIRE(in_dims % 32 == 0, GLM_ERR_UNSUPPORTED_SHAPE,
              "%s: input width %d is not a multiple of 32", who, in_dims);
  (void)fmt;
  return GLM_OK;
}

extern "C" int glm_expert_gate_up(void *stream, const uint16_t *x, int T, int d, int I, int E,
                                  int top_k, const uint8_t *gate_packed,
                                  const uint8_t *gate_scales, const uint8_t *up_packed,
                                  const uint8_t *up_scales, const int32_t *pair_token,
                                  const int32_t *work, float swiglu_limit, uint16_t *h) {
  glm::clear_error();
  GLM_REQUIRE(x && gate_packed && gate_scales && up_packed && up_scales && pair_token && work &&
                  h,
              GLM_ERR_INVALID_ARGUMENT, "expert_gate_up: null pointer argument");
  GLM_REQUIRE(T >= 0 && E >= 1 && top_k >= 1, GLM_ERR_INVALID_ARGUMENT,
              "expert_gate_up: invalid sizes");
  int rc = check_mx_geometry("expert_gate_up", GLM_FMT_MXFP4, d, I);
  if (rc) return rc;
  GLM_REQUIRE(glm_aligned16({x, gate_packed, up_packed, h, work}), GLM_ERR_INVALID_ARGUMENT,
              "expert_gate_up: buffers must be 16-byte aligned");
  if (T == 0) return GLM_OK;
  return glm_gate_up_launch((hipStream_t)stream, x, T, d, I, E, top_k, gate_packed, gate_scales,
                            up_packed, up_scales, pair_token, (const int4 *)work, swiglu_limit, h);
}

extern "C" int glm_expert_down(void *stream, const uint16_t *h, int T, int top_k, int I, int d,
                               int E, const uint8_t *down_packed, const uint8_t *down_scales,
                               const int32_t *work, uint16_t *y) {
  glm::clear_error();
  GLM_REQUIRE(h && down_packed && down_scales && work && y, GLM_ERR_INVALID_ARGUMENT,
              "expert_down: null pointer argument");
  GLM_REQUIRE(T >= 0 && E >= 1 && top_k >= 1, GLM_ERR_INVALID_ARGUMENT,
              "expert_down: invalid sizes");
  int rc = check_mx_geometry("expert_down", GLM_FMT_MXFP4, I, d);
  if (rc) return rc;
  GLM_REQUIRE(glm_aligned16({h, down_packed, y, work}), GLM_ERR_INVALID_ARGUMENT,
              "expert_down: buffers must be 16-byte aligned");
  if (T == 0) return GLM_OK;
  return glm_down_launch((hipStream_t)stream, h, T, top_k, I, d, E, down_packed, down_scales,
                         (const int4 *)work, y);
}

extern "C" int glm_linear(void *stream, const uint16_t *x, int T, int in_dims, const void *weight,
                          const uint8_t *scales, int fmt, int out_dims, uint16_t *y) {
  glm::clear_error();
  int rc = check_fmt(fmt);
  if (rc) return rc;
  GLM_REQUIRE(x && weight && y && (fmt == GLM_FMT_BF16 || scales), GLM_ERR_INVALID_ARGUMENT,
              "linear: null pointer argument");
  GLM_REQUIRE(T >= 0, GLM_ERR_INVALID_ARGUMENT, "linear: negative T");
  rc = check_mx_geometry("linear", fmt, in_dims, out_dims);
  if (rc) return rc;
  GLM_REQUIRE(glm_aligned16({x, weight, y}), GLM_ERR_INVALID_ARGUMENT,
              "linear: buffers must be 16-byte aligned");
  return glm_linear_launch((hipStream_t)stream, x, T, in_dims, weight, scales, fmt, out_dims, y);
}

extern "C" int glm_linear_f32(void *stream, const float *x, int T, int in_dims, const void *weight,
                              const uint8_t *scales, int fmt, int out_dims, uint16_t *y) {
  glm::clear_error();
  int rc = check_fmt(fmt);
  if (rc) return rc;
  GLM_REQUIRE(x && weight && y && (fmt == GLM_FMT_BF16 || scales), GLM_ERR_INVALID_ARGUMENT,
              "linear_f32: null pointer argument");
  GLM_REQUIRE(T >= 0, GLM_ERR_INVALID_ARGUMENT, "linear_f32: negative T");
  rc = check_mx_geometry("linear_f32", fmt, in_dims, out_dims);
  if (rc) return rc;
  GLM_REQUIRE(glm_aligned16({x, weight, y}), GLM_ERR_INVALID_ARGUMENT,
              "linear_f32: buffers must be 16-byte aligned");
  if (T == 0) return GLM_OK;
  GLM_REQUIRE(linear_rows_supported(T, in_dims, out_dims), GLM_ERR_UNSUPPORTED_SHAPE,
              "linear_f32: T=%d out=%d unsupported (T <= %d, out a multiple of %d)", T, out_dims,
              glm::kLinearMaxT, 4 * glm::kRowsPerWave);
  return launch_linear_rows<true>((hipStream_t)stream, x, T, in_dims, weight, scales, fmt,
                                  out_dims, y);
}

extern "C" int glm_rms_norm_linear(void *stream, const float *x, int T, int in_dims,
                                   const float *norm_weight, float eps, const void *weight,
                                   const uint8_t *scales, int fmt, int out_dims, uint16_t *y) {
  glm::clear_error();
  GLM_REQUIRE(x && weight && scales && y, GLM_ERR_INVALID_ARGUMENT,
              "rms_norm_linear: null pointer argument");
  GLM_REQUIRE(T >= 0 && eps >= 0.0f, GLM_ERR_INVALID_ARGUMENT,
              "rms_norm_linear: negative T or eps");
  GLM_REQUIRE(fmt == GLM_FMT_MXFP8, GLM_ERR_UNSUPPORTED_SHAPE,
              "rms_norm_linear: the fused norm takes MXFP8 weights (fmt %d)", fmt);
  int rc = check_mx_geometry("rms_norm_linear", fmt, in_dims, out_dims);
  if (rc) return rc;
  GLM_REQUIRE(glm_aligned16({x, weight, y, norm_weight}), GLM_ERR_INVALID_ARGUMENT,
              "rms_norm_linear: buffers must be 16-byte aligned");
  if (T == 0) return GLM_OK;
  GLM_REQUIRE(linear_rows_supported(T, in_dims, out_dims) && in_dims % 256 == 0,
              GLM_ERR_UNSUPPORTED_SHAPE,
              "rms_norm_linear: T=%d in=%d out=%d unsupported (T <= %d, in a multiple of 256, "
              "out a multiple of %d)",
              T, in_dims, out_dims, glm::kLinearMaxT, 4 * glm::kRowsPerWave);
  const glm::LinearRowsArgs a{x, T, in_dims, out_dims, static_cast<const uint8_t *>(weight),
                              scales, y, norm_weight, eps};
  hipLaunchKernelGGL((glm::linear_mx8_kernel<true, true>), dim3(out_dims / (4 * glm::kRowsPerWave)),
                     dim3(256), 0, (hipStream_t)stream, a);
  GLM_LAUNCH_CHECK("linear_mx8_kernel");
  return GLM_OK;
}

extern "C" int glm_dense_mlp(void *stream, const uint16_t *x, int T, int d, int I, int fmt,
                             const void *gate_w, const uint8_t *gate_s, const void *up_w,
                             const uint8_t *up_s, const void *down_w, const uint8_t *down_s,
                             float swiglu_limit, uint16_t *h, uint16_t *out) {
  glm::clear_error();
  int rc = check_fmt(fmt);
  if (rc) return rc;
  GLM_REQUIRE(x && gate_w && up_w && down_w && h && out, GLM_ERR_INVALID_ARGUMENT,
              "dense_mlp: null pointer argument");
  GLM_REQUIRE(fmt == GLM_FMT_BF16 || (gate_s && up_s && down_s), GLM_ERR_INVALID_ARGUMENT,
              "dense_mlp: MX weights need scales");
  GLM_REQUIRE(T >= 0, GLM_ERR_INVALID_ARGUMENT, "dense_mlp: negative T");
  rc = check_mx_geometry("dense_mlp", fmt, d, I);
  if (rc) return rc;
  rc = check_mx_geometry("dense_mlp", fmt, I, d);
  if (rc) return rc;
  GLM_REQUIRE(glm_aligned16({x, gate_w, up_w, down_w, h, out}), GLM_ERR_INVALID_ARGUMENT,
              "dense_mlp: buffers must be 16-byte aligned");
  return glm_mlp_launch((hipStream_t)stream, x, T, d, I, fmt, gate_w, gate_s, up_w, up_s, down_w,
                        down_s, swiglu_limit, h, out);
}
