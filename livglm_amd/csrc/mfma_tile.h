// Building blocks of the weight-streaming MFMA tiles (decode GEMV / skinny GEMM).
//
// A wave owns a 16-row tile of W and a K range of CPW chunks of 128.  For
// chunk c, lane (r = l & 15, q = l >> 4) holds 32 consecutive weights of row
// r -- exactly one E8M0 group -- which the gfx950 scaled converts turn into
// four bf16x8 MFMA A-fragments (values exact in bf16).  The B operand is one
// activation row per token column r at the same K positions, so
// v_mfma_f32_16x16x32_bf16 does the whole K reduction:
//   MFMA i, slot s of lane (r, q)  <->  K = kbase + 128c + 32q + 8i + s.
// MXFP4 weights (the expert bank) are stored tile-major: the 16-row x 128-K
// block (tile t, chunk c) of a matrix with K columns is 1 KB at byte
// (t K/128 + c) * 1024, lane l's 16 bytes at 16 l being row 16t + r, group
// 4c + q -- so a wave's load of one chunk reads 1 KB of contiguous memory,
// which HBM streams ~15 % faster than the 16 row pieces of the row-major
// checkpoint layout.  tile_lane_ptr gives a lane's position in the tile's
// first block; chunk c of K follows c KB further.  E8M0 scales stay
// row-major [rows][K/32].
// bf16 weights (row-major, no groups) take K = k0 + 32i + 8q + s: load i of a
// row's four lanes is then 64 contiguous bytes, and loads 2m, 2m + 1
// complete line m.
// Output lane (r, q) holds rows 4q..4q+3 of the tile for token column r.
#pragma once

#include "glm_common.h"

namespace glm {

enum { FMT_BF16 = GLM_FMT_BF16, FMT_MXFP8 = GLM_FMT_MXFP8, FMT_MXFP4 = GLM_FMT_MXFP4 };

__host__ __device__ constexpr int row_bytes(int fmt, int K) {
  return fmt == FMT_MXFP4 ? K / 2 : (fmt == FMT_MXFP8 ? K : 2 * K);
}

// Weights are streamed once: non-temporal loads keep them from evicting the
// small, reused activations and plans from the caches.
__device__ __forceinline__ glm_u32x4 load_stream(const uint8_t *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const glm_u32x4 *>(p));
}

template <int FMT>
struct WChunk;
template <>
struct WChunk<FMT_MXFP4> {
  glm_u32x4 c;
};
template <>
struct WChunk<FMT_BF16> {
  glm_u32x4 v[4];
};

// This lane's position in the first block of the 16-row tile starting at row
// row0 (a multiple of 16) of a tile-major MXFP4 matrix with K columns.
__device__ __forceinline__ const uint8_t *tile_lane_ptr(const uint8_t *w, int row0, int K,
                                                        int lane) {
  return w + (size_t)row0 * (K / 2) + 16 * lane;
}

// This lane's 32 MXFP4 weights of the chunk holding K = kl (a multiple of
// 128 plus 32q): wtile is the lane's tile_lane_ptr.
__device__ __forceinline__ WChunk<FMT_MXFP4> load_mxfp4_chunk(const uint8_t *wtile, int kl) {
  WChunk<FMT_MXFP4> w;
  w.c = load_stream(wtile + (size_t)(kl >> 7) * 1024);
  return w;
}

// bf16 weights of lane q in the chunk at k0 (row-major row wrow): K = k0 +
// 32i + 8q + [0, 8) in v[i].  NT: non-temporal loads (the full-K shared
// tiles of many tokens, whose token groups re-read a tile); otherwise plain
// loads, which the K-split tiles of a few tokens (each weight read once)
// take slightly faster: 20.8 -> 20.5-20.6 us per layer step at two tokens
// (d 2048, I_shared 768; three interleaved runs, one token within the
// spread), where plain loads in the full-K tiles measured 92.7 -> 93.3 us at
// 64 tokens.
template <bool NT = true>
__device__ __forceinline__ WChunk<FMT_BF16> load_bf16_chunk(const uint8_t *wrow, int k0, int q) {
  WChunk<FMT_BF16> w;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint8_t *p = wrow + 2 * k0 + 64 * i + 16 * q;
    w.v[i] = NT ? load_stream(p) : *reinterpret_cast<const glm_u32x4 *>(p);
  }
  return w;
}

// First K (relative to the wave's kbase) of lane q's 32 weights in chunk c.
__device__ __forceinline__ int chunk_k(int c, int q) { return c * 128 + 32 * q; }

template <int FMT>
__device__ __forceinline__ void chunk_frags(const WChunk<FMT> &w, uint32_t scale_byte,
                                            glm_bf16x8 a[4]) {
  if constexpr (FMT == FMT_MXFP4) {
    const float sc = e8m0_to_f32(scale_byte);
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = mxfp4_word_to_bf16x8(w.c[i], sc);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = __builtin_bit_cast(glm_bf16x8, w.v[i]);
  }
}

__host__ __device__ constexpr int bf16_batch(int cpw, int max_batch) {
  for (int b = max_batch; b > 1; --b)
    if (cpw % b == 0) return b;
  return 1;
}

// The MXFP4 weights of one wave (CPW chunks x NPROJ matrices): issued as one
// batch of 128-bit loads before anything that depends on the activations.
template <int FMT, int NPROJ, int CPW>
struct WaveWeights {
  static_assert(FMT == FMT_MXFP4, "tile-major MXFP4 weights");
  WChunk<FMT> w[NPROJ][CPW];
  uint32_t sd[NPROJ][CPW];  // scale dword of chunk c: byte q is lane q's group
};

// Lane q's E8M0 byte within the dword loaded for its chunk.
__device__ __forceinline__ uint32_t scale_byte(uint32_t sd, int q) { return (sd >> (8 * q)) & 0xffu; }

// wtile: each projection's tile_lane_ptr; srow: this lane's row of scales.
template <int FMT, int NPROJ, int CPW>
__device__ __forceinline__ void load_wave_weights(WaveWeights<FMT, NPROJ, CPW> &ww,
                                                  const uint8_t *const wtile[NPROJ],
                                                  const uint8_t *const srow[NPROJ], int kbase,
                                                  int q) {
  // Scales first, then the chunks in the order the MFMAs consume them: loads
  // complete in issue order, so chunk 0 can be converted while later chunks
  // are still in flight.  A scale load touches the lines of 16 rows, so the
  // CPW dwords of a row go out in as few loads as their alignment allows:
  // every caller starts a wave at a multiple of CPW chunks of rows whose
  // length is a multiple of CPW chunks, so they are 4 CPW-byte aligned.
#pragma unroll
  for (int p = 0; p < NPROJ; ++p) {
    const uint32_t *s = reinterpret_cast<const uint32_t *>(srow[p] + (kbase >> 5));
    if constexpr (CPW % 4 == 0) {
#pragma unroll
      for (int c = 0; c < CPW; c += 4) {
        const glm_u32x4 v = *reinterpret_cast<const glm_u32x4 *>(s + c);
#pragma unroll
        for (int i = 0; i < 4; ++i) ww.sd[p][c + i] = v[i];
      }
    } else if constexpr (CPW % 2 == 0) {
#pragma unroll
      for (int c = 0; c < CPW; c += 2) {
        const uint2 v = *reinterpret_cast<const uint2 *>(s + c);
        ww.sd[p][c] = v.x;
        ww.sd[p][c + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int c = 0; c < CPW; ++c) ww.sd[p][c] = s[c];
    }
  }
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) ww.w[p][c] = load_mxfp4_chunk(wtile[p], kbase + chunk_k(c, q));
  // every load above is issued before anything that follows: the scheduler
  // would otherwise sink some of them behind the first MFMAs, which costs a
  // second memory round trip
  __builtin_amdgcn_sched_barrier(0);
}

// load_wave_weights without the scale dwords: the caller fills ww.sd (for
// example from scales decoded into LDS with wave_scales_from_lds).
template <int FMT, int NPROJ, int CPW>
__device__ __forceinline__ void load_wave_chunks(WaveWeights<FMT, NPROJ, CPW> &ww,
                                                 const uint8_t *const wtile[NPROJ], int kbase,
                                                 int q) {
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) ww.w[p][c] = load_mxfp4_chunk(wtile[p], kbase + chunk_k(c, q));
  __builtin_amdgcn_sched_barrier(0);
}

// ww.sd from each projection's row of scale bytes in LDS (4-byte aligned):
// the dwords load_wave_weights reads from global memory.
template <int FMT, int NPROJ, int CPW>
__device__ __forceinline__ void wave_scales_from_lds(WaveWeights<FMT, NPROJ, CPW> &ww,
                                                     const uint8_t *const s_row[NPROJ],
                                                     int kbase, int q) {
#pragma unroll
  for (int p = 0; p < NPROJ; ++p) {
    const uint32_t *s = reinterpret_cast<const uint32_t *>(s_row[p] + (kbase >> 5));
#pragma unroll
    for (int c = 0; c < CPW; ++c) ww.sd[p][c] = s[c];
  }
}

// B fragments of this lane's 32 activations starting at K = kl.
// Activation fragments of one lane column.  `act` must point at a valid row:
// a padding column reads any valid row instead of branching (an MFMA output
// column depends only on its own B column, and padding columns are never
// stored), so the loads of every lane go out together.
__device__ __forceinline__ void load_act_frags_at(const uint16_t *act, int kl, glm_bf16x8 xb[4]) {
  const glm_bf16x8 *src = reinterpret_cast<const glm_bf16x8 *>(act + kl);
#pragma unroll
  for (int i = 0; i < 4; ++i) xb[i] = src[i];
}

// B fragments against a bf16 weight chunk at k0 (load_bf16_chunk):
// xb[i] = K k0 + 32i + 8q + [0, 8).
__device__ __forceinline__ void load_act_frags(const uint16_t *act, int k0, int q,
                                               glm_bf16x8 xb[4]) {
  const glm_bf16x8 *src = reinterpret_cast<const glm_bf16x8 *>(act + k0 + 8 * q);
#pragma unroll
  for (int i = 0; i < 4; ++i) xb[i] = src[4 * i];
}

// MFMAs of preloaded MX weights against one activation row per lane column.
template <int FMT, int NPROJ, int CPW>
__device__ __forceinline__ void mma_wave_weights(const WaveWeights<FMT, NPROJ, CPW> &ww,
                                                 int kbase, int q, const uint16_t *act,
                                                 glm_f32x4 acc[NPROJ]) {
  glm_bf16x8 xb[CPW][4];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
    load_act_frags_at(act + kbase + chunk_k(c, q), 0, xb[c]);
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
      glm_bf16x8 a[4];
      chunk_frags<FMT>(ww.w[p][c], scale_byte(ww.sd[p][c], q), a);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], xb[c][i], acc[p], 0, 0, 0);
    }
  }
}

// As mma_wave_weights, with the activation rows staged in LDS: s_row is this
// lane's token row there (nullptr: padding column).  B fragments are read per
// chunk with ds_read_b128, so registers stay free for the weight stream.
template <int FMT, int NPROJ, int CPW>
__device__ __forceinline__ void mma_wave_weights_lds(const WaveWeights<FMT, NPROJ, CPW> &ww,
                                                     int kbase, int q, const uint16_t *s_row,
                                                     glm_f32x4 acc[NPROJ]) {
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    glm_bf16x8 xb[4];
    load_act_frags_at(s_row + kbase + chunk_k(c, q), 0, xb);
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
      glm_bf16x8 a[4];
      chunk_frags<FMT>(ww.w[p][c], scale_byte(ww.sd[p][c], q), a);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], xb[i], acc[p], 0, 0, 0);
    }
  }
}

// mma_wave_weights_lds for a wave that streams several tiles through the
// same registers: right after chunk c's MFMAs the next tile's chunk c and its
// scale dword (from wtile_next / srow_next, when `next`) are issued into the
// registers they consumed, so the wave keeps about CPW chunks in flight
// across the tile boundary instead of draining to zero before the next
// tile's loads.  ww must have been filled by load_wave_weights (or by this
// function for the previous tile).
template <int FMT, int NPROJ, int CPW>
__device__ __forceinline__ void mma_wave_weights_lds_roll(
    WaveWeights<FMT, NPROJ, CPW> &ww, int kbase, int q, const uint16_t *s_row,
    glm_f32x4 acc[NPROJ], bool next, const uint8_t *const wtile_next[NPROJ],
    const uint8_t *const srow_next[NPROJ]) {
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    glm_bf16x8 xb[4];
    load_act_frags_at(s_row + kbase + chunk_k(c, q), 0, xb);
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
      glm_bf16x8 a[4];
      chunk_frags<FMT>(ww.w[p][c], scale_byte(ww.sd[p][c], q), a);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], xb[i], acc[p], 0, 0, 0);
    }
    if (next) {
#pragma unroll
      for (int p = 0; p < NPROJ; ++p) {
        ww.w[p][c] = load_mxfp4_chunk(wtile_next[p], kbase + chunk_k(c, q));
        ww.sd[p][c] = reinterpret_cast<const uint32_t *>(srow_next[p] + (kbase >> 5))[c];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// LDS row stride (bf16 elements) for staged activation rows of length K: the
// 16-byte pad spreads the rows of one MFMA B fragment over distinct banks.
__host__ __device__ constexpr int lds_row_stride(int K) { return K + 8; }

// Block-cooperative copy of `rows` activation rows of length K (bf16, K % 8
// == 0) into LDS: row j comes from src + index(j) * K, where index(j) =
// row_index[j] if row_index is given, else j.
__device__ __forceinline__ void stage_rows(uint16_t *s_x, const uint16_t *src,
                                           const int32_t *row_index, int rows, int K) {
  const int per_row = K / 8;
  for (int i = threadIdx.x; i < rows * per_row; i += blockDim.x) {
    const int j = i / per_row, c8 = i % per_row;
    const long long srow = row_index != nullptr ? row_index[j] : j;
    *reinterpret_cast<glm_u32x4 *>(s_x + j * lds_row_stride(K) + c8 * 8) =
        *reinterpret_cast<const glm_u32x4 *>(src + srow * K + c8 * 8);
  }
}

// Accumulates, over chunks [kbase/128, kbase/128 + CPW), the 16-row tile of
// NPROJ weight matrices against one activation row per lane column.  MXFP4:
// wrow is each projection's tile_lane_ptr and srow this lane's scale row
// (byte q of dword c at srow + kbase/32 is its group); bf16: wrow is this
// lane's row.  act: this lane's activation row (a valid row for a padding
// column).  NT: bf16 weights with non-temporal loads (load_bf16_chunk).
template <int FMT, int NPROJ, int CPW, bool NT = true>
__device__ __forceinline__ void wave_mma(const uint8_t *const wrow[NPROJ],
                                         const uint8_t *const srow[NPROJ], int kbase, int q,
                                         const uint16_t *act, glm_f32x4 acc[NPROJ]) {
  if constexpr (FMT != FMT_BF16) {
    WaveWeights<FMT, NPROJ, CPW> ww;
    load_wave_weights<FMT, NPROJ, CPW>(ww, wrow, srow, kbase, q);
    mma_wave_weights<FMT, NPROJ, CPW>(ww, kbase, q, act, acc);
  } else {
    // bf16 chunks are 64 B per lane: stream them in batches that divide CPW.
    constexpr int NB = bf16_batch(CPW, NPROJ == 2 ? 2 : 4);
    static_assert(CPW % NB == 0, "chunk batch must divide the chunks per wave");
#pragma unroll
    for (int b0 = 0; b0 < CPW; b0 += NB) {
      WChunk<FMT> w[NPROJ][NB];
#pragma unroll
      for (int c = 0; c < NB; ++c)
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) w[p][c] = load_bf16_chunk<NT>(wrow[p], kbase + (b0 + c) * 128, q);
      glm_bf16x8 xb[NB][4];
#pragma unroll
      for (int c = 0; c < NB; ++c) load_act_frags(act, kbase + (b0 + c) * 128, q, xb[c]);
#pragma unroll
      for (int c = 0; c < NB; ++c) {
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) {
          glm_bf16x8 a[4];
          chunk_frags<FMT>(w[p][c], 0u, a);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], xb[c][i], acc[p], 0, 0, 0);
        }
      }
    }
  }
}

// Sums the K-split partials of `nwaves` waves in fixed wave order through LDS
// (red: (nwaves - 1) * NPROJ * 64 float4; wave 0 keeps its own in registers).  Returns true on the wave that holds the
// total (wave 0); the block must call it uniformly.
template <int NPROJ>
__device__ __forceinline__ bool ksplit_reduce(glm_f32x4 acc[NPROJ], glm_f32x4 *red, int wave,
                                              int nwaves, int lane) {
  if (nwaves == 1) return true;
  if (wave > 0) {
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) red[((wave - 1) * NPROJ + p) * 64 + lane] = acc[p];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
      glm_f32x4 s = acc[p];
      for (int w = 1; w < nwaves; ++w) s += red[((w - 1) * NPROJ + p) * 64 + lane];
      acc[p] = s;
    }
  }
  __syncthreads();
  return wave == 0;
}

// Stores lane (r, q)'s four rows 4q..4q+3 (bf16) of token column r.
__device__ __forceinline__ void store_rows4(uint16_t *dst, const uint32_t o[4]) {
  uint2 packed;
  packed.x = o[0] | (o[1] << 16);
  packed.y = o[2] | (o[3] << 16);
  *reinterpret_cast<uint2 *>(dst) = packed;
}

}  // namespace glm
