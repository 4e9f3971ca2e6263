// Token-to-expert dispatch: histogram -> exclusive prefix sum -> stable permute.
//
// The reference materialises routes on the host once per layer (unique +
// compact remap, native_expert_ssd.py:475-525; expert_ssd.py:159-169).  Here
// the grouping stays on the device: pairs p = t*k + j are counting-sorted by
// expert id, ties kept in ascending p, so each expert's rows are contiguous
// for the expert kernels.
#include <algorithm>

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

// Row tiles of the grouped GEMMs: an expert's c rows go to
// nt = ceil(c / tile_rows) tiles (tile_rows a multiple of 16), its 16-row
// blocks dealt out evenly, so every tile but the last is a whole number of
// blocks and none exceeds tile_rows (ceil(c / 16) <= nt * tile_rows / 16).
// Tile i is {first row within the expert, rows}.
__device__ __forceinline__ int row_tiles(int c, int tile_rows) {
  return (c + tile_rows - 1) / tile_rows;
}
__device__ __forceinline__ int2 row_tile(int c, int nt, int i) {
  const long long blocks = (c + 15) / 16;
  const int r0 = 16 * (int)(i * blocks / nt);
  const int r1 = min(16 * (int)((i + 1) * blocks / nt), c);
  return make_int2(r0, r1 - r0);
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
  // optionally the row tiles of the grouped GEMMs (row_tile, in expert
  // order): {expert, first sorted position, rows, 0}.
  int carry = 0, carry_active = 0, carry_tiles = 0;
  for (int e0 = 0; e0 < E; e0 += kDispatchThreads) {
    const int e = e0 + tid;
    const int c = e < E ? (int)cnt[e] : 0;
    int tot = 0;
    const int ex = block_exclusive_scan(c, s_scan, &tot);
    int tot_a = 0;
    const int ex_a = block_exclusive_scan(c > 0 ? 1 : 0, s_scan, &tot_a);
    const int nt = tiles != nullptr ? row_tiles(c, tile_rows) : 0;
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
      for (int i = 0; i < nt; ++i) {
        const int2 t = row_tile(c, nt, i);
        tiles[carry_tiles + ex_t + i] = make_int4(e, carry + ex + t.x, t.y, 0);
      }
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
  // positions past the valid pairs (dropped indices >= E) hold -1
  for (int pos = carry + tid; pos < P; pos += kDispatchThreads) {
    perm[pos] = -1;
    pair_token[pos] = -1;
  }
}

// ---------------------------------------------------------------------------
// Multi-workgroup dispatch for many pairs: the pairs are cut into chunks of
// 1024 (one workgroup each).  (1) every chunk counts its experts (done by the
// scan's own workgroup when the chunk histograms fit its LDS); (2) one
// workgroup turns the chunk counts into expert offsets and per-chunk bases
// (bases[c][e] = offsets[e] + pairs of expert e in chunks < c), plus the work
// list and row tiles; (3) every chunk ranks its pairs stably within the chunk
// (bitmap popcount, as above) and scatters them to bases[c][e] + rank.  The
// result is identical to the single-workgroup dispatch.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kDispatchThreads) void dispatch_count_kernel(
    const uint32_t *__restrict__ idx, int P, int E, int32_t *__restrict__ chunk_counts) {
  extern __shared__ uint32_t cnt[];  // [E]
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += kDispatchThreads) cnt[e] = 0;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  const int p = blockIdx.x * kDispatchThreads + tid;
  if (p < P) {
    const uint32_t e = idx[p];
    if (e < (uint32_t)E) atomicAdd(&cnt[e], 1u);
    else s_bad = 1;
  }
  __syncthreads();
  int32_t *row = chunk_counts + (size_t)blockIdx.x * (E + 1);
  for (int e = tid; e < E; e += kDispatchThreads) row[e] = (int)cnt[e];
  if (tid == 0) row[E] = s_bad;
}

// FUSED: the same workgroup first counts the chunks itself, into LDS
// histograms [nchunks][E] (dynamic LDS), reading the indices once; the chunk
// bases then go to chunk_counts for the scatter as in the three-kernel form.
template <bool FUSED>
__global__ __launch_bounds__(kDispatchThreads) void dispatch_scan_kernel(
    const uint32_t *__restrict__ idx, int P, int32_t *__restrict__ chunk_counts, int nchunks,
    int E, int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
    int32_t *__restrict__ active, int32_t *__restrict__ num_active, int4 *__restrict__ work,
    int32_t *__restrict__ status, int tile_rows, int4 *__restrict__ tiles,
    int32_t *__restrict__ num_tiles) {
  extern __shared__ int32_t hist[];  // FUSED: [nchunks][E]
  __shared__ int s_scan[kDispatchThreads / 64 + 1];
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  int bad = 0;
  if constexpr (FUSED) {
    for (int i = tid; i < nchunks * E; i += kDispatchThreads) hist[i] = 0;
    if (tid == 0) s_bad = 0;
    __syncthreads();
    // thread t takes pair t of every chunk, 16 chunks' loads at a time
    for (int c0 = 0; c0 < nchunks; c0 += 16) {
      uint32_t ev[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const long long p = (long long)(c0 + j) * kDispatchThreads + tid;
        ev[j] = c0 + j < nchunks && p < P ? idx[p] : 0xffffffffu;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const long long p = (long long)(c0 + j) * kDispatchThreads + tid;
        if (c0 + j < nchunks && p < P) {
          if (ev[j] < (uint32_t)E) atomicAdd(&hist[(c0 + j) * E + ev[j]], 1);
          else s_bad = 1;
        }
      }
    }
    __syncthreads();
    bad = s_bad;
  } else {
    // bad flags OR-ed by thread 0
    if (tid == 0)
      for (int c = 0; c < nchunks; ++c) bad |= chunk_counts[(size_t)c * (E + 1) + E];
  }
  // per expert: running sum over chunks (the count of chunk c becomes the
  // exclusive base of chunk c within the expert)
  int carry = 0, carry_active = 0, carry_tiles = 0;
  for (int e0 = 0; e0 < E; e0 += kDispatchThreads) {
    const int e = e0 + tid;
    int c_e = 0;
    if (e < E) {
      // 16 chunks at a time: their loads are issued together before any store
      for (int c0 = 0; c0 < nchunks; c0 += 16) {
        int n[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
          n[j] = c0 + j >= nchunks ? 0
                 : FUSED           ? hist[(c0 + j) * E + e]
                                   : chunk_counts[(size_t)(c0 + j) * (E + 1) + e];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          if (c0 + j < nchunks) {
            if (FUSED)
              hist[(c0 + j) * E + e] = c_e;
            else
              chunk_counts[(size_t)(c0 + j) * (E + 1) + e] = c_e;
          }
          c_e += n[j];
        }
      }
    }
    int tot = 0;
    const int ex = block_exclusive_scan(c_e, s_scan, &tot);
    int tot_a = 0;
    const int ex_a = block_exclusive_scan(c_e > 0 ? 1 : 0, s_scan, &tot_a);
    const int nt = tiles != nullptr ? row_tiles(c_e, tile_rows) : 0;
    int tot_t = 0;
    const int ex_t = block_exclusive_scan(nt, s_scan, &tot_t);
    if (e < E) {
      const int off = carry + ex;
      offsets[e] = off;
      counts[e] = c_e;
      for (int c0 = 0; c0 < nchunks; c0 += 16) {
        int v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
          v[j] = c0 + j >= nchunks ? 0
                 : FUSED           ? hist[(c0 + j) * E + e]
                                   : chunk_counts[(size_t)(c0 + j) * (E + 1) + e];
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (c0 + j < nchunks) chunk_counts[(size_t)(c0 + j) * (E + 1) + e] = v[j] + off;
      }
      if (c_e > 0) {
        active[carry_active + ex_a] = e;
        work[carry_active + ex_a] = make_int4(e, off, c_e, 0);
      }
      for (int i = 0; i < nt; ++i) {
        const int2 t = row_tile(c_e, nt, i);
        tiles[carry_tiles + ex_t + i] = make_int4(e, off + t.x, t.y, 0);
      }
    }
    carry += tot;
    carry_active += tot_a;
    carry_tiles += tot_t;
  }
  if (tid == 0) {
    offsets[E] = carry;
    num_active[0] = carry_active;
    status[0] = bad;
    if (num_tiles != nullptr) num_tiles[0] = carry_tiles;
  }
  for (int e = carry_active + tid; e < E; e += kDispatchThreads) {
    active[e] = -1;
    work[e] = make_int4(-1, 0, 0, 0);
  }
}

__global__ __launch_bounds__(kDispatchThreads) void dispatch_scatter_kernel(
    const uint32_t *__restrict__ idx, int P, int k, int E,
    const int32_t *__restrict__ chunk_bases, int32_t *__restrict__ perm,
    int32_t *__restrict__ inv, int32_t *__restrict__ pair_token) {
  extern __shared__ uint32_t bits[];  // [E][32]
  const int tid = threadIdx.x;
  for (int w = tid; w < E * 32; w += kDispatchThreads) bits[w] = 0;
  __syncthreads();
  const int p = blockIdx.x * kDispatchThreads + tid;
  uint32_t e = 0xffffffffu;
  if (p < P) {
    e = idx[p];
    if (e < (uint32_t)E) atomicOr(&bits[e * 32 + (tid >> 5)], 1u << (tid & 31));
  }
  __syncthreads();
  if (p < P) {
    if (e < (uint32_t)E) {
      const uint32_t *row = bits + e * 32;
      int r = chunk_bases[(size_t)blockIdx.x * (E + 1) + e];
      const int word = tid >> 5;
      for (int w = 0; w < word; ++w) r += __popc(row[w]);
      r += __popc(row[word] & ((1u << (tid & 31)) - 1u));
      perm[r] = p;
      inv[p] = r;
      if (pair_token != nullptr) pair_token[r] = p / k;
    } else {
      inv[p] = -1;
    }
  }
}

// pair_token from perm once the scatter is done (the public dispatch keeps
// the chunk counts in pair_token until then); positions past the valid pairs
// hold -1 in both.
__global__ void dispatch_tokens_kernel(const int32_t *__restrict__ offsets, int E, int P, int k,
                                       int32_t *__restrict__ perm,
                                       int32_t *__restrict__ pair_token) {
  const int total = offsets[E];
  for (int pos = blockIdx.x * blockDim.x + threadIdx.x; pos < P; pos += gridDim.x * blockDim.x) {
    if (pos < total) {
      pair_token[pos] = perm[pos] / k;
    } else {
      perm[pos] = -1;
      pair_token[pos] = -1;
    }
  }
}

// Row tiles of the grouped GEMMs from a work list (one workgroup): slot u of
// {expert, first position, rows, 0} gives row_tiles(rows, tile_rows) tiles.
__global__ __launch_bounds__(kDispatchThreads) void tiles_from_work_kernel(
    const int4 *__restrict__ work, int E, int tile_rows, int4 *__restrict__ tiles,
    int32_t *__restrict__ num_tiles) {
  __shared__ int s_scan[kDispatchThreads / 64 + 1];
  const int tid = threadIdx.x;
  int carry = 0;
  for (int u0 = 0; u0 < E; u0 += kDispatchThreads) {
    const int u = u0 + tid;
    const int4 wk = u < E ? work[u] : make_int4(-1, 0, 0, 0);
    const int n = wk.x >= 0 ? wk.z : 0;
    const int nt = row_tiles(n, tile_rows);
    int tot = 0;
    const int ex = block_exclusive_scan(nt, s_scan, &tot);
    for (int i = 0; i < nt; ++i) {
      const int2 t = row_tile(n, nt, i);
      tiles[carry + ex + i] = make_int4(wk.x, wk.y + t.x, t.y, 0);
    }
    carry += tot;
  }
  if (tid == 0) num_tiles[0] = carry;
}

}  // namespace glm

int glm_grouped_tile_rows();

extern "C" int glm_moe_tiles(void *stream, const int32_t *work, int E, int32_t *tiles,
                             int32_t *num_tiles) {
  glm::clear_error();
  GLM_REQUIRE(work && tiles && num_tiles, GLM_ERR_INVALID_ARGUMENT, "moe_tiles: null pointer");
  GLM_REQUIRE(E >= 1, GLM_ERR_INVALID_ARGUMENT, "moe_tiles: invalid E=%d", E);
  GLM_REQUIRE(glm_aligned16({work, tiles}), GLM_ERR_INVALID_ARGUMENT,
              "moe_tiles: work and tiles must be 16-byte aligned");
  hipLaunchKernelGGL(glm::tiles_from_work_kernel, dim3(1), dim3(glm::kDispatchThreads), 0,
                     (hipStream_t)stream, reinterpret_cast<const int4 *>(work), E,
                     glm_grouped_tile_rows(), reinterpret_cast<int4 *>(tiles), num_tiles);
  GLM_LAUNCH_CHECK("tiles_from_work_kernel");
  return GLM_OK;
}

size_t glm_dispatch_lds_bytes(int E) { return (size_t)E * (3 + 32) * sizeof(uint32_t); }

// Pairs above which the dispatch runs on many workgroups (it then needs
// glm_dispatch_chunk_ints(P, E) ints of scratch).
constexpr int kMultiDispatchPairs = 4096;
size_t glm_dispatch_chunk_ints(long long P, int E) {
  return P > kMultiDispatchPairs
             ? (size_t)((P + glm::kDispatchThreads - 1) / glm::kDispatchThreads) * (E + 1)
             : 0;
}

// tiles/num_tiles (optional): row tiles of tile_rows rows for the grouped
// GEMMs; tiles needs room for ceil(T*k / tile_rows) + E entries.
// chunk_scratch: glm_dispatch_chunk_ints(P, E) ints for the multi-workgroup
// dispatch; without it (the public entry point) the chunk counts live in
// pair_token -- ceil(P / 1024) * (E + 1) <= P ints for E <= 448 and P > 4096
// -- and pair_token is filled from perm at the end.
int glm_dispatch_launch(hipStream_t stream, const uint32_t *indices, int T, int k, int E,
                        int32_t *counts, int32_t *offsets, int32_t *perm, int32_t *inv,
                        int32_t *pair_token, int32_t *active, int32_t *num_active, int4 *work,
                        int32_t *status, int tile_rows, int4 *tiles, int32_t *num_tiles,
                        int32_t *chunk_scratch) {
  const int P = T * k;
  if (P > kMultiDispatchPairs) {
    const int nchunks = (P + glm::kDispatchThreads - 1) / glm::kDispatchThreads;
    const bool in_place = chunk_scratch == nullptr;
    if (in_place) {
      GLM_REQUIRE((size_t)nchunks * (E + 1) <= (size_t)P, GLM_ERR_UNSUPPORTED_SHAPE,
                  "dispatch: %d chunks x %d experts do not fit in pair_token", nchunks, E + 1);
      chunk_scratch = pair_token;
    }
    // the chunk histograms of one workgroup fit its LDS up to 64 KB (T*k
    // pairs x E experts: 131,072 x 128): count and scan in one kernel
    const size_t hist_bytes = (size_t)nchunks * E * 4;
    if (hist_bytes <= 64 * 1024) {
      hipLaunchKernelGGL(glm::dispatch_scan_kernel<true>, dim3(1), dim3(glm::kDispatchThreads),
                         hist_bytes, stream, indices, P, chunk_scratch, nchunks, E, counts,
                         offsets, active, num_active, work, status, tile_rows, tiles, num_tiles);
      GLM_LAUNCH_CHECK("dispatch_scan_kernel");
    } else {
      hipLaunchKernelGGL(glm::dispatch_count_kernel, dim3(nchunks), dim3(glm::kDispatchThreads),
                         (size_t)E * 4, stream, indices, P, E, chunk_scratch);
      GLM_LAUNCH_CHECK("dispatch_count_kernel");
      hipLaunchKernelGGL(glm::dispatch_scan_kernel<false>, dim3(1), dim3(glm::kDispatchThreads),
                         0, stream, indices, P, chunk_scratch, nchunks, E, counts, offsets,
                         active, num_active, work, status, tile_rows, tiles, num_tiles);
      GLM_LAUNCH_CHECK("dispatch_scan_kernel");
    }
    hipLaunchKernelGGL(glm::dispatch_scatter_kernel, dim3(nchunks), dim3(glm::kDispatchThreads),
                       (size_t)E * 32 * 4, stream, indices, P, k, E, chunk_scratch, perm, inv,
                       in_place ? nullptr : pair_token);
    GLM_LAUNCH_CHECK("dispatch_scatter_kernel");
    if (in_place) {
      const int blocks = std::min((P + 255) / 256, 1024);
      hipLaunchKernelGGL(glm::dispatch_tokens_kernel, dim3(blocks), dim3(256), 0, stream, offsets,
                         E, P, k, perm, pair_token);
      GLM_LAUNCH_CHECK("dispatch_tokens_kernel");
    }
    return GLM_OK;
  }
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
                             nullptr, nullptr, nullptr);
}
