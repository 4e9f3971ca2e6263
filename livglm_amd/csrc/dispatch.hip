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
// 1024 (one workgroup each), in two kernels that run on every chunk at once.
// (1) dispatch_rank_kernel: every chunk ranks its pairs stably within the
// chunk -- lanes of a wave with the same expert are found with one ballot per
// bit of the expert id, a pair's rank is the number of such lanes below it
// plus the same expert's pairs in the chunk's earlier waves (per-wave counts
// in LDS) -- and writes its expert counts.  (2) dispatch_place_kernel: every
// chunk sums the chunk counts itself (expert totals and the counts of the
// chunks before it), scans the totals into expert offsets and places its
// pairs at offset + earlier chunks + rank; chunk 0 also writes the offsets,
// counts, work list and row tiles.  The result is identical to the
// single-workgroup dispatch.
// ---------------------------------------------------------------------------
constexpr int kDispatchWaves = kDispatchThreads / 64;

// LDS: per-wave expert counts [kDispatchWaves][E] (E <= 448).
__global__ __launch_bounds__(kDispatchThreads) void dispatch_rank_kernel(
    const uint32_t *__restrict__ idx, int P, int E, int32_t *__restrict__ chunk_counts,
    int32_t *__restrict__ local_rank) {
  extern __shared__ int32_t wcnt[];  // [kDispatchWaves][E]
  __shared__ int s_bad;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kDispatchWaves * E; i += kDispatchThreads) wcnt[i] = 0;
  if (tid == 0) s_bad = 0;
  const int p = blockIdx.x * kDispatchThreads + tid;
  const uint32_t e = p < P ? idx[p] : (uint32_t)E;
  // key E stands for "no pair" (past the end, or an index >= E, which is dropped)
  const uint32_t key = e < (uint32_t)E ? e : (uint32_t)E;
  __syncthreads();
  if (p < P && e >= (uint32_t)E) s_bad = 1;
  // the lanes holding this lane's key: one ballot per bit of the key
  const int nbits = 32 - __clz(E);
  uint64_t same = ~0ull;
  for (int bit = 0; bit < nbits; ++bit) {
    const uint64_t m = __ballot((key >> bit) & 1u);
    same &= ((key >> bit) & 1u) ? m : ~m;
  }
  const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
  if (key < (uint32_t)E && below == 0) wcnt[wave * E + key] = __popcll(same);
  __syncthreads();
  // per expert: exclusive prefix over the waves; the chunk's count
  for (int x = tid; x < E; x += kDispatchThreads) {
    int run = 0;
#pragma unroll
    for (int w = 0; w < kDispatchWaves; ++w) {
      const int c = wcnt[w * E + x];
      wcnt[w * E + x] = run;
      run += c;
    }
    chunk_counts[(size_t)blockIdx.x * (E + 1) + x] = run;
  }
  __syncthreads();
  if (tid == 0) chunk_counts[(size_t)blockIdx.x * (E + 1) + E] = s_bad;
  if (p < P) local_rank[p] = key < (uint32_t)E ? wcnt[wave * E + key] + below : -1;
}

// rank_inv: in, the chunk-local ranks of dispatch_rank_kernel; out, inv.
// pair_token may be null (then the caller fills it from perm).
__global__ __launch_bounds__(kDispatchThreads) void dispatch_place_kernel(
    const uint32_t *__restrict__ idx, int P, int k, int E,
    const int32_t *__restrict__ chunk_counts, int nchunks, int32_t *__restrict__ rank_inv,
    int32_t *__restrict__ perm, int32_t *__restrict__ pair_token, int32_t *__restrict__ counts,
    int32_t *__restrict__ offsets, int32_t *__restrict__ active, int32_t *__restrict__ num_active,
    int4 *__restrict__ work, int32_t *__restrict__ status, int tile_rows,
    int4 *__restrict__ tiles, int32_t *__restrict__ num_tiles) {
  __shared__ int32_t base[448];
  __shared__ int s_scan[kDispatchThreads / 64 + 1];
  const int tid = threadIdx.x;
  const int chunk = blockIdx.x;
  // expert tid: its total over all chunks and its pairs in the chunks before
  // this one (16 chunks' loads issued together)
  int total = 0, before = 0;
  if (tid < E) {
    for (int c0 = 0; c0 < nchunks; c0 += 16) {
      int n[16];
#pragma unroll
      for (int j = 0; j < 16; ++j)
        n[j] = c0 + j < nchunks ? chunk_counts[(size_t)(c0 + j) * (E + 1) + tid] : 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        total += n[j];
        before += c0 + j < chunk ? n[j] : 0;
      }
    }
  }
  int all = 0;
  const int off = block_exclusive_scan(tid < E ? total : 0, s_scan, &all);
  if (tid < E) base[tid] = off + before;
  __syncthreads();
  const int p = chunk * kDispatchThreads + tid;
  if (p < P) {
    const uint32_t e = idx[p];
    const int r = rank_inv[p];
    if (e < (uint32_t)E && r >= 0) {
      const int pos = base[e] + r;
      perm[pos] = p;
      rank_inv[p] = pos;
      if (pair_token != nullptr) pair_token[pos] = p / k;
    } else {
      rank_inv[p] = -1;
    }
  }
  if (chunk != 0) return;
  // chunk 0: offsets, counts, the work list of active experts, row tiles
  int tot_a = 0;
  const int ex_a = block_exclusive_scan(tid < E && total > 0 ? 1 : 0, s_scan, &tot_a);
  const int nt = tiles != nullptr && tid < E ? row_tiles(total, tile_rows) : 0;
  int tot_t = 0;
  const int ex_t = block_exclusive_scan(nt, s_scan, &tot_t);
  if (tid < E) {
    offsets[tid] = off;
    counts[tid] = total;
    if (total > 0) {
      active[ex_a] = tid;
      work[ex_a] = make_int4(tid, off, total, 0);
    }
    for (int i = 0; i < nt; ++i) {
      const int2 t = row_tile(total, nt, i);
      tiles[ex_t + i] = make_int4(tid, off + t.x, t.y, 0);
    }
  }
  for (int x = tot_a + tid; x < E; x += kDispatchThreads) {
    active[x] = -1;
    work[x] = make_int4(-1, 0, 0, 0);
  }
  // positions past the valid pairs (dropped indices >= E) hold -1
  for (int pos = all + tid; pos < P; pos += kDispatchThreads) {
    perm[pos] = -1;
    if (pair_token != nullptr) pair_token[pos] = -1;
  }
  int bad = 0;
  for (int c = tid; c < nchunks; c += kDispatchThreads) bad |= chunk_counts[(size_t)c * (E + 1) + E];
  bad = __syncthreads_or(bad);
  if (tid == 0) {
    offsets[E] = all;
    num_active[0] = tot_a;
    status[0] = bad ? 1 : 0;
    if (num_tiles != nullptr) num_tiles[0] = tot_t;
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
    // the chunk-local ranks go through inv, which the second kernel overwrites
    hipLaunchKernelGGL(glm::dispatch_rank_kernel, dim3(nchunks), dim3(glm::kDispatchThreads),
                       (size_t)glm::kDispatchWaves * E * 4, stream, indices, P, E, chunk_scratch,
                       inv);
    GLM_LAUNCH_CHECK("dispatch_rank_kernel");
    hipLaunchKernelGGL(glm::dispatch_place_kernel, dim3(nchunks), dim3(glm::kDispatchThreads), 0,
                       stream, indices, P, k, E, chunk_scratch, nchunks, inv, perm,
                       in_place ? nullptr : pair_token, counts, offsets, active, num_active, work,
                       status, tile_rows, tiles, num_tiles);
    GLM_LAUNCH_CHECK("dispatch_place_kernel");
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
