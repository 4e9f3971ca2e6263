// Prefill grouped GEMMs of the routed experts on gfx950 MFMA.
//
// For every routed expert e with n_e > 0 rows in dispatch (sorted) order
// (native_expert_ssd.py:726-743 runs gather_qmm over all (t, j) pairs):
//   gate/up: h[pos] = limited_swiglu(bf16(x[tok(pos)] . Wg_e^T), bf16(x[tok(pos)] . Wu_e^T))
//   down:    y[pos] = bf16(h[pos] . Wd_e^T)
// The dispatch cuts each expert's rows into tiles of kTileM rows.  A workgroup
// computes one row tile against kTileW = 256 weight rows (gate/up: 128
// features of each projection; down: 256 features) in a 4 x 2
// arrangement of eight waves: wave (wf, wt) owns 64 weight rows x 64 tokens,
// i.e. 4 x 4 accumulator tiles of v_mfma_f32_16x16x32_bf16 (two waves per
// SIMD, so one wave's conversions and LDS reads overlap the other's MFMAs).  K advances in chunks of 128:
// the activation rows (bf16, gathered through the dispatch for gate/up) and
// the weight rows (packed MXFP4 + E8M0 scales) of a chunk are staged in LDS,
// double-buffered, and the next chunk's global loads are issued before the
// current chunk's MFMAs.  Weights are converted to bf16 in registers with
// v_cvt_scalef32_pk_bf16_fp4 (exact for the checkpoints' scales).
//
// K mapping (as in the decode tiles): MFMA i of chunk c, slot s of lane (r, q)
// is K = 128c + 32q + 8i + s -- lane q's 16 staged bytes of a weight row are one
// whole E8M0 group, so each lane needs one scale byte per chunk.
#include "mfma_tile.h"

namespace glm {

constexpr int kTileM = 128;            // token rows per tile
constexpr int kChunkK = 128;           // K per stage
constexpr int kXStride = kChunkK + 8;  // staged activation row, bf16 elements
constexpr int kWStride = 80;           // staged weight row, bytes (64 B of codes + pad)

// Weight rows per workgroup for RT row tiles per wave (4 waves along the rows).
__host__ __device__ constexpr int tile_w(int RT) { return RT * 64; }
__host__ __device__ constexpr int stage_bytes(int RT) {
  return kTileM * kXStride * 2 + tile_w(RT) * kWStride + tile_w(RT) * 4;
}

struct GroupedArgs {
  const uint16_t *act;       // gate/up: x [T][K]; down: h [P][K]
  const int32_t *act_index;  // sorted position -> activation row (nullptr: the position)
  const int4 *tiles;         // {expert, first sorted position, rows, 0}
  const int32_t *num_tiles;
  const uint8_t *w[2];       // stacked codes [E][N][K/2] per projection
  const uint8_t *s[2];       // stacked E8M0 scales [E][N][K/32]
  long long w_stride, s_stride;
  int N, K;                  // weight rows per expert and projection; reduction length
  int feature_tiles;         // workgroups along N per row tile
  uint16_t *out;             // bf16 [P][N]
  float limit;               // bf16-rounded SwiGLU limit (gate/up)
};

// Workgroup -> (row tile, feature tile), XCD-aware: workgroups are dealt to
// the 8 XCDs round-robin by linear id, so XCD x takes the x-th contiguous
// eighth of the work items, ordered row tile major.  The feature tiles of one
// row tile (which share its activation rows) and the row tiles of one expert
// (which share its weights) then run side by side on one XCD and meet in its
// L2.  Items past the real tile count (known only on the device) exit.
constexpr int kXcds = 8;

constexpr int kThreads = 512;  // 8 waves: 4 along the weight rows x 2 along the tokens

template <int NPROJ, int RT>
__global__ __launch_bounds__(kThreads) void grouped_mx_gemm_kernel(GroupedArgs a) {
  constexpr int kTileW = tile_w(RT);
  constexpr int kStageBytes = stage_bytes(RT);
  constexpr int HALF = RT / 2;  // gate/up: row tiles per projection per wave
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nft = a.feature_tiles;
  const int items = *a.num_tiles * nft;
  const int lin = blockIdx.x;  // the grid is a multiple of kXcds covering every item
  const int per_xcd = (items + kXcds - 1) / kXcds;
  const int k_on_xcd = lin / kXcds;
  const int item = (lin % kXcds) * per_xcd + k_on_xcd;
  if (k_on_xcd >= per_xcd || item >= items) return;
  const int tile_id = item / nft, ftile = item % nft;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int wf = wave & 3, wt = wave >> 2;
  const int4 tile = a.tiles[tile_id];
  const long long e = tile.x;
  const int pos0 = tile.y, rows = tile.z;
  const int K = a.K;
  const int nchunks = K / kChunkK;
  // weight rows of this workgroup: NPROJ == 2 -> [gate f0..f0+127 | up f0..f0+127]
  const int f0 = ftile * (kTileW / NPROJ);

  // ---- staging assignment (fixed over the K loop)
  // activations: piece j = row (tid >> 4) + 32 j, 16 bytes at column (tid & 15).
  // Rows past the tile's end re-read its first row: MFMA columns are
  // independent and those columns are never stored.
  const uint16_t *xsrc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = (tid >> 4) + 32 * j;
    const int pos = pos0 + (row < rows ? row : 0);
    const long long arow = a.act_index != nullptr ? a.act_index[pos] : pos;
    xsrc[j] = a.act + arow * K + (tid & 15) * 8;
  }
  // weights: piece j = row (tid >> 2) + 128 j, 16 bytes at (tid & 3); scales:
  // row tid < kTileW
  constexpr int WP = kTileW / 128;  // weight pieces per thread
  const uint8_t *wsrc[WP];
#pragma unroll
  for (int j = 0; j < WP; ++j) {
    const int wrow = (tid >> 2) + 128 * j;
    const int p = NPROJ == 2 ? wrow / (kTileW / 2) : 0;
    const int frow = f0 + (NPROJ == 2 ? wrow % (kTileW / 2) : wrow);
    wsrc[j] = a.w[p] + e * a.w_stride + (size_t)frow * (K / 2) + (tid & 3) * 16;
  }
  const uint8_t *ssrc;
  {
    const int srow = tid & (kTileW - 1);
    const int p = NPROJ == 2 ? srow / (kTileW / 2) : 0;
    const int frow = f0 + (NPROJ == 2 ? srow % (kTileW / 2) : srow);
    ssrc = a.s[p] + e * a.s_stride + (size_t)frow * (K / 32);
  }

  glm_u32x4 stx[4], stw[WP];
  uint32_t sts = 0;
  auto load_stage = [&](int c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) stx[j] = *reinterpret_cast<const glm_u32x4 *>(xsrc[j] + c * kChunkK);
#pragma unroll
    for (int j = 0; j < WP; ++j) stw[j] = load_stream(wsrc[j] + c * (kChunkK / 2));
    if (tid < kTileW) sts = *reinterpret_cast<const uint32_t *>(ssrc + c * (kChunkK / 32));
  };
  auto store_stage = [&](int buf) {
    uint8_t *base = smem + buf * kStageBytes;
    uint16_t *sx = reinterpret_cast<uint16_t *>(base);
    uint8_t *sw = base + kTileM * kXStride * 2;
    uint32_t *ss = reinterpret_cast<uint32_t *>(sw + kTileW * kWStride);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<glm_u32x4 *>(sx + ((tid >> 4) + 32 * j) * kXStride + (tid & 15) * 8) = stx[j];
#pragma unroll
    for (int j = 0; j < WP; ++j)
      *reinterpret_cast<glm_u32x4 *>(sw + ((tid >> 2) + 128 * j) * kWStride + (tid & 3) * 16) = stw[j];
    if (tid < kTileW) ss[tid] = sts;
  };

  glm_f32x4 acc[RT][4];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = glm_f32x4{0.f, 0.f, 0.f, 0.f};

  // this wave's RT weight-row tiles within the staged rows (gate/up: RT/2 gate
  // tiles, then the up tiles of the same features)
  auto wrow_of = [&](int rt) {
    return NPROJ == 2 ? (rt / HALF) * (kTileW / 2) + wf * HALF * 16 + (rt % HALF) * 16
                      : wf * RT * 16 + rt * 16;
  };

  // MFMAs of one staged chunk
  auto compute = [&](int buf) {
    const uint8_t *base = smem + buf * kStageBytes;
    const uint16_t *sx = reinterpret_cast<const uint16_t *>(base);
    const uint8_t *sw = base + kTileM * kXStride * 2;
    const uint32_t *ss = reinterpret_cast<const uint32_t *>(sw + kTileW * kWStride);
    glm_u32x4 raw[RT];
    float scale[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int wr = wrow_of(rt) + r;
      raw[rt] = *reinterpret_cast<const glm_u32x4 *>(sw + wr * kWStride + 16 * q);
      scale[rt] = e8m0_to_f32((ss[wr] >> (8 * q)) & 0xffu);
    }
    // every B fragment of the chunk is read up front (LDS returns in order, so
    // the MFMAs of step i wait only for the reads of steps <= i)
    glm_bf16x8 xb[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        xb[i][ct] = *reinterpret_cast<const glm_bf16x8 *>(sx + (wt * 64 + ct * 16 + r) * kXStride +
                                                          32 * q + 8 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const glm_bf16x8 af = mxfp4_word_to_bf16x8(raw[rt][i], scale[rt]);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, xb[i][ct], acc[rt][ct], 0, 0, 0);
      }
    }
  };

  load_stage(0);
  store_stage(0);
  __syncthreads();
  // steady state: next chunk's loads in flight during this chunk's MFMAs; the
  // last chunk is peeled so the loop body has no conditional work
  for (int c = 0; c + 1 < nchunks; ++c) {
    load_stage(c + 1);
    compute(c & 1);
    store_stage((c + 1) & 1);
    __syncthreads();
  }
  compute((nchunks - 1) & 1);

  // ---- epilogue: lane (r, q) of tile (rt, ct) holds features 4q..4q+3 of the
  // row tile for token column r
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int row = wt * 64 + ct * 16 + r;
    if (row >= rows) continue;
    uint16_t *orow = a.out + (size_t)(pos0 + row) * a.N;
    if constexpr (NPROJ == 2) {
#pragma unroll
      for (int i = 0; i < HALF; ++i) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
          o[m] = f32_to_bf16(limited_swiglu(bf16_round(acc[i][ct][m]),
                                            bf16_round(acc[HALF + i][ct][m]), a.limit));
        store_rows4(orow + f0 + wf * HALF * 16 + i * 16 + 4 * q, o);
      }
    } else {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = f32_to_bf16(acc[rt][ct][m]);
        store_rows4(orow + f0 + wf * RT * 16 + rt * 16 + 4 * q, o);
      }
    }
  }
}

}  // namespace glm

using namespace glm;

int glm_grouped_tile_rows() { return kTileM; }

// Whether the grouped GEMMs cover these shapes: gate/up K = d, N = I in
// feature tiles of 128 per projection; down K = I, N = d in tiles of 256.
bool glm_grouped_supported(int d, int I) {
  return d % kChunkK == 0 && I % kChunkK == 0 && I % 128 == 0 && d % 256 == 0;
}

static int grouped_launch(hipStream_t stream, GroupedArgs a, int nproj, int max_tiles) {
  constexpr int rt = 4;  // 8 row tiles per wave would need more than 256 registers
  a.feature_tiles = a.N / (nproj == 2 ? tile_w(rt) / 2 : tile_w(rt));
  // XCD x handles items [x * per, (x + 1) * per) with per <= ceil(max_items / 8),
  // at linear ids x + 8k: the grid must reach 8 * ceil(max_items / 8)
  const long long max_items = (long long)max_tiles * a.feature_tiles;
  const dim3 grid((unsigned)(((max_items + kXcds - 1) / kXcds) * kXcds));
  const size_t lds = 2 * (size_t)stage_bytes(rt);
  if (nproj == 2)
    hipLaunchKernelGGL((grouped_mx_gemm_kernel<2, rt>), grid, dim3(kThreads), lds, stream, a);
  else
    hipLaunchKernelGGL((grouped_mx_gemm_kernel<1, rt>), grid, dim3(kThreads), lds, stream, a);
  GLM_LAUNCH_CHECK("grouped_mx_gemm_kernel");
  return GLM_OK;
}

int glm_grouped_gate_up_launch(hipStream_t stream, const uint16_t *x, const int32_t *pair_token,
                               const int4 *tiles, const int32_t *num_tiles, int max_tiles, int d,
                               int I, const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                               const uint8_t *us, uint16_t *h, float limit) {
  GroupedArgs a{};
  a.act = x;
  a.act_index = pair_token;
  a.tiles = tiles;
  a.num_tiles = num_tiles;
  a.w[0] = gw;
  a.w[1] = uw;
  a.s[0] = gs;
  a.s[1] = us;
  a.w_stride = (long long)I * (d / 2);
  a.s_stride = (long long)I * (d / 32);
  a.N = I;
  a.K = d;
  a.out = h;
  a.limit = glm_limit_bf16(limit);
  return grouped_launch(stream, a, 2, max_tiles);
}

int glm_grouped_down_launch(hipStream_t stream, const uint16_t *h, const int4 *tiles,
                            const int32_t *num_tiles, int max_tiles, int I, int d,
                            const uint8_t *dw, const uint8_t *ds, uint16_t *y) {
  GroupedArgs a{};
  a.act = h;
  a.act_index = nullptr;
  a.tiles = tiles;
  a.num_tiles = num_tiles;
  a.w[0] = a.w[1] = dw;
  a.s[0] = a.s[1] = ds;
  a.w_stride = (long long)d * (I / 2);
  a.s_stride = (long long)d * (I / 32);
  a.N = d;
  a.K = I;
  a.out = y;
  return grouped_launch(stream, a, 1, max_tiles);
}
