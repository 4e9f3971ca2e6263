// Token-to-expert dispatch: histogram -> exclusive prefix sum -> stable permute.
//
// The reference materialises routes on the host once per layer (unique +
// compact remap, native_expert_ssd.py:475-525; expert_ssd.py:159-169).  Here
// the grouping stays on the device: pairs p = t*k + j are counting-sorted by
// expert id, ties kept in ascending p, so each expert's rows are contiguous
// for the expert kernels.
#include "glm_common.h"

namespace glm {

constexpr int kDispatchThreads = 1024;

// Exclusive scan of one value per thread over a 1024-thread block.  Returns
// the exclusive prefix; *total receives the block sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int *s_wave, int *total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) s_wave[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kDispatchThreads / 64 ? s_wave[lane] : 0;
    int wi = w;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(wi, off, 64);
      if (lane >= off) wi += o;
    }
    if (lane < kDispatchThreads / 64) s_wave[lane] = wi - w;  // exclusive wave base
    if (lane == kDispatchThreads / 64 - 1) s_wave[kDispatchThreads / 64] = wi;
  }
  __syncthreads();
  const int base = s_wave[wave];
  *total = s_wave[kDispatchThreads / 64];
  __syncthreads();
  return base + incl - v;
}

// Single workgroup; LDS: cnt[E] off[E] run[E] bits[E][32] + scan scratch.
__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(
    const uint32_t *__restrict__ idx, int P, int k, int E, int32_t *__restrict__ counts,
    int32_t *__restrict__ offsets, int32_t *__restrict__ perm, int32_t *__restrict__ inv,
    int32_t *__restrict__ pair_token, int32_t *__restrict__ active,
    int32_t *__restrict__ num_active, int4 *__restrict__ work, int32_t *__restrict__ status,
    int tile_rows, int4 *__restrict__ tiles, int32_t *__restrict__ num_tiles) {
  extern __shared__ uint32_t smem[];
  uint32_t *cnt = smem;
  uint32_t *off = cnt + E;
  uint32_t *run = off + E;
  uint32_t *bits = run + E;  // [E][32]: one bit per pair of the current 1024-pair chunk
  __shared__ int s_scan[kDispatchThreads / 64 + 1];
  __shared__ int s_bad;
  const int tid = threadIdx.x;

  for (int e = tid; e < E; e += kDispatchThreads) {
    cnt[e] = 0;
    run[e] = 0;
  }
  if (tid == 0) s_bad = 0;
  __syncthreads();
  for (int p = tid; p < P; p += kDispatchThreads) {
    const uint32_t e = idx[p];
    if (e < (uint32_t)E) atomicAdd(&cnt[e], 1u);
    else s_bad = 1;
  }
  __syncthreads();

  // offsets = exclusive scan of counts; active = compacted ids with count > 0;
  // optionally the row tiles of the grouped GEMMs (tile_rows rows each, in
  // expert order): {expert, first sorted position, rows, 0}.
  int carry = 0, carry_active = 0, carry_tiles = 0;
  for (int e0 = 0; e0 < E; e0 += kDispatchThreads) {
    const int e = e0 + tid;
    const int c = e < E ? (int)cnt[e] : 0;
    int tot = 0;
    const int ex = block_exclusive_scan(c, s_scan, &tot);
    int tot_a = 0;
    const int ex_a = block_exclusive_scan(c > 0 ? 1 : 0, s_scan, &tot_a);
    const int nt = tiles != nullptr ? (c + tile_rows - 1) / tile_rows : 0;
    int tot_t = 0;
    const int ex_t = block_exclusive_scan(nt, s_scan, &tot_t);
    if (e < E) {
      off[e] = carry + ex;
      offsets[e] = carry + ex;
      counts[e] = c;
      if (c > 0) {
        active[carry_active + ex_a] = e;
        work[carry_active + ex_a] = make_int4(e, carry + ex, c, 0);
      }
      for (int i = 0; i < nt; ++i)
        tiles[carry_tiles + ex_t + i] =
            make_int4(e, carry + ex + i * tile_rows, min(tile_rows, c - i * tile_rows), 0);
    }
    carry += tot;
    carry_active += tot_a;
    carry_tiles += tot_t;
  }
  if (tid == 0) {
    offsets[E] = carry;
    num_active[0] = carry_active;
    status[0] = s_bad;
    if (num_tiles != nullptr) num_tiles[0] = carry_tiles;
  }
  for (int e = carry_active + tid; e < E; e += kDispatchThreads) {
    active[e] = -1;
    work[e] = make_int4(-1, 0, 0, 0);
  }
  __syncthreads();

  // Stable ranks, one 1024-pair chunk at a time: rank(p) = run[e] + number
  // of earlier pairs of this chunk with the same expert (bitmap popcount).
  for (int p0 = 0; p0 < P; p0 += kDispatchThreads) {
    for (int w = tid; w < E * 32; w += kDispatchThreads) bits[w] = 0;
    __syncthreads();
    const int p = p0 + tid;
    uint32_t e = 0xffffffffu;
    if (p < P) {
      e = idx[p];
      if (e < (uint32_t)E) atomicOr(&bits[e * 32 + (tid >> 5)], 1u << (tid & 31));
    }
    __syncthreads();
    if (p < P) {
      if (e < (uint32_t)E) {
        const uint32_t *row = bits + e * 32;
        uint32_t r = run[e];
        const int word = tid >> 5;
        for (int w = 0; w < word; ++w) r += __popc(row[w]);
        r += __popc(row[word] & ((1u << (tid & 31)) - 1u));
        const int pos = (int)(off[e] + r);
        perm[pos] = p;
        inv[p] = pos;
        pair_token[pos] = p / k;
      } else {
        inv[p] = -1;
      }
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += kDispatchThreads) {
      uint32_t c = 0;
      for (int w = 0; w < 32; ++w) c += __popc(bits[ee * 32 + w]);
      run[ee] += c;
    }
    __syncthreads();
  }
}

}  // namespace glm

size_t glm_dispatch_lds_bytes(int E) { return (size_t)E * (3 + 32) * sizeof(uint32_t); }

// tiles/num_tiles (optional): row tiles of tile_rows rows for the grouped
// GEMMs; tiles needs room for ceil(T*k / tile_rows) + E entries.
int glm_dispatch_launch(hipStream_t stream, const uint32_t *indices, int T, int k, int E,
                        int32_t *counts, int32_t *offsets, int32_t *perm, int32_t *inv,
                        int32_t *pair_token, int32_t *active, int32_t *num_active, int4 *work,
                        int32_t *status, int tile_rows, int4 *tiles, int32_t *num_tiles) {
  const int P = T * k;
  hipLaunchKernelGGL(glm::dispatch_kernel, dim3(1), dim3(glm::kDispatchThreads),
                     glm_dispatch_lds_bytes(E), stream, indices, P, k, E, counts, offsets, perm,
                     inv, pair_token, active, num_active, work, status, tile_rows, tiles,
                     num_tiles);
  GLM_LAUNCH_CHECK("dispatch_kernel");
  return GLM_OK;
}

extern "C" int glm_moe_dispatch(void *stream, const uint32_t *indices, int T, int top_k, int E,
                                int32_t *counts, int32_t *offsets, int32_t *perm, int32_t *inv,
                                int32_t *pair_token, int32_t *active, int32_t *num_active,
                                int32_t *work, int32_t *status) {
  glm::clear_error();
  GLM_REQUIRE(indices && counts && offsets && perm && inv && pair_token && active &&
                  num_active && work && status,
              GLM_ERR_INVALID_ARGUMENT, "dispatch: null pointer argument");
  GLM_REQUIRE(T >= 0 && top_k >= 1 && E >= 1, GLM_ERR_INVALID_ARGUMENT,
              "dispatch: invalid sizes T=%d k=%d E=%d", T, top_k, E);
  GLM_REQUIRE(E <= 448, GLM_ERR_UNSUPPORTED_SHAPE, "dispatch: E=%d exceeds 448", E);
  GLM_REQUIRE((long long)T * top_k < (1LL << 30), GLM_ERR_UNSUPPORTED_SHAPE,
              "dispatch: too many pairs");
  GLM_REQUIRE(glm_aligned16({work}), GLM_ERR_INVALID_ARGUMENT,
              "dispatch: work must be 16-byte aligned");
  return glm_dispatch_launch((hipStream_t)stream, indices, T, top_k, E, counts, offsets, perm,
                             inv, pair_token, active, num_active, (int4 *)work, status, 0,
                             nullptr, nullptr);
}
