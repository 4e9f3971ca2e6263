// In-kernel decode of ScaleX Mode-B scale rows (scale_codec.py:34-201,
// docs/scalex-mode-b.md:24-33): the routed expert kernels read an expert's
// E8M0 scales from its coded row and decode the rows of their tile into LDS
// while its weights stream in.
//
// An expert's row holds its Mode-B form (encode_mode_b_row,
// scale_codec.py:150-154) with the tile directory in front, so that the
// directory and the record's header sit at fixed offsets and arrive in one
// round trip:
//   [0, dir_bytes)   u16 directory: entry t = index of the first exception at
//                    or past scale 512 t ((raw + 511) / 512 + 1 entries), zero
//                    padding to a multiple of 16 bytes;
//   [dir_bytes, ..)  the Mode-A record of the expert's gate | down | up scale
//                    bytes: a 24-byte header (magic, codec, four palette bytes,
//                    3 pad, raw size, primary size, exception count), the
//                    primary codes (codec 1: one bit per scale, codec 2: two
//                    bits, codec 0: the raw bytes; LSB first), the exception
//                    positions (u32 little-endian, ascending) and values (u8).
#pragma once

#include "glm_common.h"

namespace glm {

// Bytes of a row's directory (with its padding) for `raw` scale bytes.
__host__ __device__ constexpr uint32_t scalex_dir_bytes(uint32_t raw) {
  return ((2 * ((raw + 511) / 512 + 1)) + 15) / 16 * 16;
}

struct ScalexRow {
  const uint16_t *dir;
  const uint8_t *rec;
  uint32_t codec, palette, primary, nexc;
};

// The directory and the record header of a row (16-byte aligned).
__device__ __forceinline__ ScalexRow scalex_row(const uint8_t *row, uint32_t dir_bytes) {
  ScalexRow h;
  h.dir = reinterpret_cast<const uint16_t *>(row);
  h.rec = row + dir_bytes;
  const uint32_t *w = reinterpret_cast<const uint32_t *>(h.rec);
  const uint32_t w1 = w[1], w2 = w[2];
  h.codec = w1 & 0xffu;
  h.palette = (w1 >> 8) | (w2 << 24);
  h.primary = w[4];
  h.nexc = w[5];
  return h;
}

__device__ __forceinline__ uint32_t scalex_pal(uint32_t palette, uint32_t code) {
  return (palette >> (8 * code)) & 0xffu;
}

__device__ __forceinline__ uint32_t scalex_load_u32(const uint8_t *p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

// The primary codes of 32 scales [p, p + 32) (p % 4 == 0) of a row coded
// with CODEC: codec 1 the 32 one-bit codes in c[0]; codec 2 the 64 two-bit
// codes in c[0] (first 16) and c[1]; raw the bytes in c[0..7] (word j =
// scales p + 4j ..).  Branch-free: every address is clamped into the primary
// codes (codecs 1, 2) or the range's `cnt` scales (raw), and the bytes past
// them read as 0, so the loads of all ranges go out before any is waited on.
template <int CODEC>
__device__ __forceinline__ void scalex_load32(const ScalexRow &h, uint32_t p, uint32_t cnt,
                                              uint32_t c[8]) {
  const uint8_t *prim = h.rec + 24;
  if constexpr (CODEC == 1) {
    // bits p .. p + 31 lie in bytes p/8 .. p/8 + 4 (bit p at bit p % 8 of the first)
    const uint32_t b0 = p >> 3;
    uint64_t win = 0;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      const uint32_t v = prim[min(b0 + i, h.primary - 1)];
      win |= (uint64_t)(b0 + i < h.primary ? v : 0u) << (8 * i);
    }
    c[0] = (uint32_t)(win >> (p & 7));
  } else if constexpr (CODEC == 2) {
    // codes of scales p .. p + 31: bytes p/4 .. p/4 + 7 (p % 4 == 0: whole bytes)
    const uint32_t b0 = p >> 2;
    c[0] = c[1] = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t v = prim[min(b0 + i, h.primary - 1)];
      c[i >> 2] |= (b0 + i < h.primary ? v : 0u) << (8 * (i & 3));
    }
  } else {
    // raw bytes (24 + p is 4-aligned); cnt >= 4
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = *reinterpret_cast<const uint32_t *>(prim + p + min(4u * j, cnt - 4));
  }
}

// Word j (scales 4j .. 4j + 3 of the 32) of codes loaded by scalex_load32.
template <int CODEC>
__device__ __forceinline__ uint32_t scalex_word32(const ScalexRow &h, const uint32_t c[8], int j) {
  if constexpr (CODEC == 1) {
    const uint32_t b = (c[0] >> (4 * j)) & 0xfu;  // four one-bit codes
    return scalex_pal(h.palette, b & 1) | scalex_pal(h.palette, (b >> 1) & 1) << 8 |
           scalex_pal(h.palette, (b >> 2) & 1) << 16 | scalex_pal(h.palette, b >> 3) << 24;
  } else if constexpr (CODEC == 2) {
    const uint32_t b = (c[j >> 2] >> (8 * (j & 3))) & 0xffu;  // four two-bit codes
    return scalex_pal(h.palette, b & 3) | scalex_pal(h.palette, (b >> 2) & 3) << 8 |
           scalex_pal(h.palette, (b >> 4) & 3) << 16 | scalex_pal(h.palette, b >> 6) << 24;
  } else {
    return c[j];
  }
}

// scalex_decode for one codec (below).
template <int CODEC, int R, typename Sync>
__device__ __forceinline__ void scalex_decode_codec(const ScalexRow &h, const uint32_t s0[R],
                                                    uint32_t n, uint8_t *const dst[R], int tid,
                                                    int nthreads, Sync sync, const uint32_t e0[R],
                                                    const uint32_t e1[R]) {
  const uint8_t *pos = h.rec + 24 + h.primary;
  const uint8_t *val = pos + 4 * h.nexc;
  for (uint32_t b = 32 * (uint32_t)tid; b < n; b += 32 * (uint32_t)nthreads) {
    const uint32_t cnt = min(32u, n - b);
    uint32_t c[R][8];
#pragma unroll
    for (int i = 0; i < R; ++i) scalex_load32<CODEC>(h, s0[i] + b, cnt, c[i]);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      uint32_t *d = reinterpret_cast<uint32_t *>(dst[i] + b);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (4u * j < cnt) d[j] = scalex_word32<CODEC>(h, c[i], j);
    }
  }
  // each thread's first exception of each range, loaded after the codes
  uint32_t p1[R], v1[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t u = e0[i] + tid;
    p1[i] = 0xffffffffu;
    v1[i] = 0;
    if (u < e1[i]) {
      p1[i] = scalex_load_u32(pos + 4 * u);
      v1[i] = val[u];
    }
  }
  sync();  // the primary bytes are down before exceptions overwrite them
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (p1[i] >= s0[i] && p1[i] < s0[i] + n) dst[i][p1[i] - s0[i]] = (uint8_t)v1[i];
    // more exceptions than threads in the range: further rounds
    for (uint32_t u = e0[i] + tid + nthreads; u < e1[i]; u += nthreads) {
      const uint32_t p = scalex_load_u32(pos + 4 * u);
      if (p >= s0[i] && p < s0[i] + n) dst[i][p - s0[i]] = val[u];
    }
  }
}

// Decodes, for each of the R ranges i, scales [s0[i], s0[i] + n) of row h
// into dst[i] (LDS, 4-byte aligned; s0[i] % 4 == 0, n % 4 == 0, n > 0), with
// the threads tid = 0..nthreads-1 of the group that sync() synchronises (the
// row's codec is the same for all of them).  Each thread takes 32
// consecutive scales of every range per pass (one pass when n <= 32 nthreads:
// every shape the expert kernels use); the directory entries are read with
// the header, then all the codes of a pass are loaded at once, and the first
// exception of each range per thread; the primary bytes are written, then,
// after sync(), the exceptions over them.  Ends without a final sync: the
// caller synchronises before reading dst.
template <int R, typename Sync>
__device__ __forceinline__ void scalex_decode(const ScalexRow &h, const uint32_t s0[R],
                                              uint32_t n, uint8_t *const dst[R], int tid,
                                              int nthreads, Sync sync) {
  uint32_t e0[R], e1[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    e0[i] = h.dir[s0[i] / 512];
    e1[i] = h.dir[(s0[i] + n - 1) / 512 + 1];
  }
  if (h.codec == 1)
    scalex_decode_codec<1, R>(h, s0, n, dst, tid, nthreads, sync, e0, e1);
  else if (h.codec == 2)
    scalex_decode_codec<2, R>(h, s0, n, dst, tid, nthreads, sync, e0, e1);
  else
    scalex_decode_codec<0, R>(h, s0, n, dst, tid, nthreads, sync, e0, e1);
}

}  // namespace glm
