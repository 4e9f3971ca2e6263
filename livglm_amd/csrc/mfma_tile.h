// Building blocks of the weight-streaming MFMA tiles (decode GEMV / skinny GEMM).
//
// A wave owns a 16-row tile of W and a K range of CPW chunks of 128.  For
// chunk c, lane (r = l & 15, q = l >> 4) holds 32 consecutive weights of row
// r -- exactly one E8M0 group -- which the gfx950 scaled converts turn into
// four bf16x8 MFMA A-fragments (values exact in bf16).  The B operand is one
// activation row per token column r at the same K positions, so
// v_mfma_f32_16x16x32_bf16 does the whole K reduction:
//   MFMA i, slot s of lane (r, q)  <->  K = kbase + chunk_k(c, q) + 8i + s.
// chunk_k is c*128 + 32q, except for MXFP4 with an even chunk count, where
// chunks pair up as (c>>1)*256 + 64q + 32(c&1): the four lanes of a row then
// read one whole 128-byte line per chunk pair (two 16-byte loads each) rather
// than half a line per load, which the memory system serves faster.
// bf16 weights (no groups) take K = k0 + 32i + 8q + s: load i of a row's four
// lanes is then 64 contiguous bytes, and loads 2m, 2m + 1 complete line m.
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
struct WChunk<FMT_MXFP8> {
  glm_u32x4 c0, c1;
};
template <>
struct WChunk<FMT_BF16> {
  glm_u32x4 v[4];
};

// The 32 MX weights of this lane starting at K = kl (one E8M0 group).
template <int FMT>
__device__ __forceinline__ WChunk<FMT> load_chunk_at(const uint8_t *wrow, int kl) {
  static_assert(FMT != FMT_BF16, "MX weights");
  WChunk<FMT> w;
  if constexpr (FMT == FMT_MXFP4) {
    w.c = load_stream(wrow + (kl >> 1));
  } else {
    w.c0 = load_stream(wrow + kl);
    w.c1 = load_stream(wrow + kl + 16);
  }
  return w;
}

// Lane q's weights of the chunk at k0: MX, the group K [k0 + 32q, k0 + 32q +
// 32); bf16, K = k0 + 32i + 8q + [0, 8) in v[i].
template <int FMT>
__device__ __forceinline__ WChunk<FMT> load_chunk(const uint8_t *wrow, int k0, int q) {
  if constexpr (FMT == FMT_BF16) {
    WChunk<FMT> w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w.v[i] = load_stream(wrow + 2 * k0 + 64 * i + 16 * q);
    return w;
  } else {
    return load_chunk_at<FMT>(wrow, k0 + 32 * q);
  }
}

template <int FMT, int CPW>
__host__ __device__ constexpr bool paired_chunks() {
  return FMT == FMT_MXFP4 && CPW % 2 == 0;
}

// First K (relative to the wave's kbase) of lane q's 32 weights in chunk c.
template <int FMT, int CPW>
__device__ __forceinline__ int chunk_k(int c, int q) {
  if constexpr (paired_chunks<FMT, CPW>())
    return (c >> 1) * 256 + 64 * q + 32 * (c & 1);
  else
    return c * 128 + 32 * q;
}

template <int FMT>
__device__ __forceinline__ void chunk_frags(const WChunk<FMT> &w, uint32_t scale_byte,
                                            glm_bf16x8 a[4]) {
  if constexpr (FMT == FMT_MXFP4) {
    const float sc = e8m0_to_f32(scale_byte);
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = mxfp4_word_to_bf16x8(w.c[i], sc);
  } else if constexpr (FMT == FMT_MXFP8) {
    const float sc = e8m0_to_f32(scale_byte);
    a[0] = mxfp8_words_to_bf16x8(w.c0[0], w.c0[1], sc);
    a[1] = mxfp8_words_to_bf16x8(w.c0[2], w.c0[3], sc);
    a[2] = mxfp8_words_to_bf16x8(w.c1[0], w.c1[1], sc);
    a[3] = mxfp8_words_to_bf16x8(w.c1[2], w.c1[3], sc);
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

// The MX weights of one wave (CPW chunks x NPROJ matrices): issued as one
// batch of 128-bit loads before anything that depends on the activations.
template <int FMT, int NPROJ, int CPW>
struct WaveWeights {
  WChunk<FMT> w[NPROJ][CPW];
  uint32_t sd[NPROJ][CPW];  // scale dword holding lane q's group of chunk c (see scale_byte)
};

// Lane q's E8M0 byte of chunk c within the dword loaded for it.
template <int FMT, int CPW>
__device__ __forceinline__ uint32_t scale_byte(uint32_t sd, int c, int q) {
  if constexpr (paired_chunks<FMT, CPW>())
    return (sd >> (8 * (2 * (q & 1) + (c & 1)))) & 0xffu;
  else
    return (sd >> (8 * q)) & 0xffu;
}

template <int FMT, int NPROJ, int CPW>
__device__ __forceinline__ void load_wave_weights(WaveWeights<FMT, NPROJ, CPW> &ww,
                                                  const uint8_t *const wrow[NPROJ],
                                                  const uint8_t *const srow[NPROJ], int kbase,
                                                  int q) {
  static_assert(FMT != FMT_BF16, "bf16 weights are streamed in batches by wave_mma");
  // Scales first, then the chunks in the order the MFMAs consume them: loads
  // complete in issue order, so chunk 0 can be converted while later chunks
  // are still in flight.
#pragma unroll
  for (int p = 0; p < NPROJ; ++p) {
    const uint32_t *s = reinterpret_cast<const uint32_t *>(srow[p] + (kbase >> 5));
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      if constexpr (paired_chunks<FMT, CPW>()) {
        // groups of chunk pair m: 8 bytes at m*8; lane q's two are bytes 2q, 2q+1
        if ((c & 1) == 0) ww.sd[p][c] = s[(c >> 1) * 2 + (q >> 1)];
        else ww.sd[p][c] = ww.sd[p][c - 1];
      } else {
        ww.sd[p][c] = s[c];
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int p = 0; p < NPROJ; ++p)
      ww.w[p][c] = load_chunk_at<FMT>(wrow[p], kbase + chunk_k<FMT, CPW>(c, q));
  // every load above is issued before anything that follows: the scheduler
  // would otherwise sink some of them behind the first MFMAs, which costs a
  // second memory round trip
  __builtin_amdgcn_sched_barrier(0);
}

// load_wave_weights without the scale dwords: the caller fills ww.sd (for
// example from scales decoded into LDS with wave_scales_from_lds).
template <int FMT, int NPROJ, int CPW>
__device__ __forceinline__ void load_wave_chunks(WaveWeights<FMT, NPROJ, CPW> &ww,
                                                 const uint8_t *const wrow[NPROJ], int kbase,
                                                 int q) {
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int p = 0; p < NPROJ; ++p)
      ww.w[p][c] = load_chunk_at<FMT>(wrow[p], kbase + chunk_k<FMT, CPW>(c, q));
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
    for (int c = 0; c < CPW; ++c) {
      if constexpr (paired_chunks<FMT, CPW>())
        ww.sd[p][c] = s[(c >> 1) * 2 + (q >> 1)];
      else
        ww.sd[p][c] = s[c];
    }
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

// B fragments against a bf16 weight chunk at k0 (load_chunk<FMT_BF16>):
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
    load_act_frags_at(act + kbase + chunk_k<FMT, CPW>(c, q), 0, xb[c]);
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
      glm_bf16x8 a[4];
      chunk_frags<FMT>(ww.w[p][c], scale_byte<FMT, CPW>(ww.sd[p][c], c, q), a);
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
    load_act_frags_at(s_row + kbase + chunk_k<FMT, CPW>(c, q), 0, xb);
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
      glm_bf16x8 a[4];
      chunk_frags<FMT>(ww.w[p][c], scale_byte<FMT, CPW>(ww.sd[p][c], c, q), a);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], xb[i], acc[p], 0, 0, 0);
    }
  }
}

// mma_wave_weights_lds for a wave that streams several tiles through the
// same registers: right after chunk c's MFMAs the next tile's chunk c (from
// wrow_next / srow_next, when `next`) is issued into the registers they
// consumed, so the wave keeps about CPW chunks in flight across the tile
// boundary instead of draining to zero before the next tile's loads.  With
// paired chunks the scale dword of pair m serves chunks 2m and 2m + 1; the
// next tile's dword goes out after chunk 2m + 1's MFMAs.  ww must have been
// filled by load_wave_weights (or by this function for the previous tile).
template <int FMT, int NPROJ, int CPW>
__device__ __forceinline__ void mma_wave_weights_lds_roll(
    WaveWeights<FMT, NPROJ, CPW> &ww, int kbase, int q, const uint16_t *s_row,
    glm_f32x4 acc[NPROJ], bool next, const uint8_t *const wrow_next[NPROJ],
    const uint8_t *const srow_next[NPROJ]) {
  static_assert(FMT != FMT_BF16, "MX weights");
  constexpr bool kPaired = paired_chunks<FMT, CPW>();
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    glm_bf16x8 xb[4];
    load_act_frags_at(s_row + kbase + chunk_k<FMT, CPW>(c, q), 0, xb);
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
      glm_bf16x8 a[4];
      const uint32_t sd = kPaired ? ww.sd[p][c & ~1] : ww.sd[p][c];
      chunk_frags<FMT>(ww.w[p][c], scale_byte<FMT, CPW>(sd, c, q), a);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], xb[i], acc[p], 0, 0, 0);
    }
    if (next) {
#pragma unroll
      for (int p = 0; p < NPROJ; ++p) {
        ww.w[p][c] = load_chunk_at<FMT>(wrow_next[p], kbase + chunk_k<FMT, CPW>(c, q));
        const uint32_t *sn = reinterpret_cast<const uint32_t *>(srow_next[p] + (kbase >> 5));
        if constexpr (kPaired) {
          if (c & 1) ww.sd[p][c & ~1] = sn[(c >> 1) * 2 + (q >> 1)];
        } else {
          ww.sd[p][c] = sn[c];
        }
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
// NPROJ weight matrices against one activation row per lane column.
// wrow/srow: this lane's weight/scale row; act: this lane's activation row
// (nullptr for a padding column).  Scales of the CPW chunks are CPW aligned
// dwords at srow + kbase/32 (byte q of dword c is this lane's group).
template <int FMT, int NPROJ, int CPW>
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
        for (int p = 0; p < NPROJ; ++p) w[p][c] = load_chunk<FMT>(wrow[p], kbase + (b0 + c) * 128, q);
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
