// Prefill grouped GEMMs of the routed experts (and the dense shared expert)
// on gfx950 MFMA.
//
// For every routed expert e with n_e > 0 rows in dispatch (sorted) order
// (native_expert_ssd.py:726-743 runs gather_qmm over all (t, j) pairs):
//   gate/up: h[pos] = limited_swiglu(bf16(x[tok(pos)] . Wg_e^T), bf16(x[tok(pos)] . Wu_e^T))
//   down:    y[pos] = bf16(h[pos] . Wd_e^T)
// and, in dense mode (one "expert", rows = tokens), the bf16 shared expert
// DenseMLP (layers.py:160-171) at many tokens.
//
// The dispatch cuts each expert's rows into tiles of kTileM rows.  A workgroup
// computes one row tile against kTileW = 256 weight rows (gate/up: 128
// features of each projection; down: 256 features) in a 4 x 2 arrangement of
// eight waves: wave (wf, wt) owns 64 weight rows x 64 tokens, i.e. 4 x 4
// accumulator tiles of v_mfma_f32_16x16x32_bf16 (two waves per SIMD, so one
// wave's conversions and LDS reads overlap the other's MFMAs).  K advances in
// chunks (128 for MXFP4 weights, 64 for bf16): the activation rows (bf16,
// gathered through the dispatch for gate/up) and the weight rows of a chunk
// are staged in LDS, double-buffered, and the next chunk's global loads are
// issued before the current chunk's MFMAs.  MXFP4 weights are converted to
// bf16 in registers with v_cvt_scalef32_pk_bf16_fp4 (exact for the
// checkpoints' scales).
//
// K mapping.  MXFP4: MFMA i of a chunk, slot s of lane (r, q) is K = 32q + 8i +
// s -- lane q's 16 staged bytes of a weight row are one whole E8M0 group, so
// each lane needs one scale byte per chunk.  bf16: K = 32i + 8q + s (natural).
//
// Workgroup -> (row tile, feature tile) is XCD-aware: workgroups are dealt to
// the 8 XCDs round-robin by linear id, so XCD x takes the x-th contiguous
// eighth of the work items, ordered row tile major.  The feature tiles of one
// row tile (which share its activation rows) and the row tiles of one expert
// (which share its weights) then run side by side on one XCD and meet in its
// L2.  Items past the real tile count (known only on the device) exit.
#include "mfma_tile.h"

namespace glm {

constexpr int kTileM = 128;    // token rows per tile
constexpr int kTileW = 256;    // weight rows per workgroup
constexpr int kThreads = 512;  // 8 waves: 4 along the weight rows x 2 along the tokens
constexpr int kXcds = 8;

template <int WFMT>
struct GroupedLayout {
  static constexpr int kChunk = WFMT == FMT_MXFP4 ? 128 : 64;  // K per stage
  static constexpr int kXStride = kChunk + 8;                  // staged activation row, bf16
  static constexpr int kWRowBytes = WFMT == FMT_MXFP4 ? kChunk / 2 : kChunk * 2;
  static constexpr int kWStride = kWRowBytes + 16;             // staged weight row, bytes
  static constexpr int kXBytes = kTileM * kXStride * 2;
  static constexpr int kWBytes = kTileW * kWStride;
  static constexpr int kSBytes = WFMT == FMT_MXFP4 ? kTileW * 4 : 0;
  static constexpr int kStageBytes = kXBytes + kWBytes + kSBytes;
  static constexpr int kXPerRow = kChunk / 8;  // 16-byte pieces per staged row
  static constexpr int kWPerRow = kWRowBytes / 16;
  static constexpr int kXPieces = kTileM * kXPerRow / kThreads;  // pieces per thread
  static constexpr int kWPieces = kTileW * kWPerRow / kThreads;
};

struct GroupedArgs {
  const uint16_t *act;       // gate/up: x [T][K]; down: h [P][K]
  const int32_t *act_index;  // sorted position -> activation row (nullptr: the position)
  const int4 *tiles;         // {expert, first sorted position, rows, 0}
  const int32_t *num_tiles;
  int dense_rows;            // > 0: dense mode, tiles of kTileM consecutive rows of expert 0
  const uint8_t *w[2];       // stacked weights [E][N][row bytes] per projection
  const uint8_t *s[2];       // stacked E8M0 scales [E][N][K/32] (MXFP4)
  long long w_stride, s_stride;
  int N, K;                  // weight rows per expert and projection; reduction length
  int feature_tiles;         // workgroups along N per row tile
  uint16_t *out;             // bf16 [rows][N]
  float limit;               // bf16-rounded SwiGLU limit (gate/up)
};

template <int NPROJ, int WFMT>
__global__ __launch_bounds__(kThreads) void grouped_mx_gemm_kernel(GroupedArgs a) {
  using L = GroupedLayout<WFMT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nft = a.feature_tiles;
  const int ntiles = a.dense_rows > 0 ? (a.dense_rows + kTileM - 1) / kTileM : *a.num_tiles;
  const int items = ntiles * nft;
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
  const int4 tile =
      a.dense_rows > 0
          ? make_int4(0, tile_id * kTileM, min(kTileM, a.dense_rows - tile_id * kTileM), 0)
          : a.tiles[tile_id];
  const long long e = tile.x;
  const int pos0 = tile.y, rows = tile.z;
  const int K = a.K;
  const int nchunks = K / L::kChunk;
  // weight rows of this workgroup: NPROJ == 2 -> [gate f0..f0+127 | up f0..f0+127]
  const int f0 = ftile * (kTileW / NPROJ);
  const int wrow_bytes = WFMT == FMT_MXFP4 ? K / 2 : K * 2;

  // ---- staging assignment (fixed over the K loop)
  // activations: piece j = row tid / kXPerRow + j * (kThreads / kXPerRow), 16
  // bytes at column tid % kXPerRow.  Rows past the tile's end re-read its first
  // row: MFMA columns are independent and those columns are never stored.
  const uint16_t *xsrc[L::kXPieces];
#pragma unroll
  for (int j = 0; j < L::kXPieces; ++j) {
    const int row = tid / L::kXPerRow + j * (kThreads / L::kXPerRow);
    const int pos = pos0 + (row < rows ? row : 0);
    const long long arow = a.act_index != nullptr ? a.act_index[pos] : pos;
    xsrc[j] = a.act + arow * K + (tid % L::kXPerRow) * 8;
  }
  // weights: piece j = row tid / kWPerRow + j * (kThreads / kWPerRow); scales: row tid < kTileW
  const uint8_t *wsrc[L::kWPieces];
#pragma unroll
  for (int j = 0; j < L::kWPieces; ++j) {
    const int wrow = tid / L::kWPerRow + j * (kThreads / L::kWPerRow);
    const int p = NPROJ == 2 ? wrow / (kTileW / 2) : 0;
    const int frow = f0 + (NPROJ == 2 ? wrow % (kTileW / 2) : wrow);
    wsrc[j] = a.w[p] + e * a.w_stride + (size_t)frow * wrow_bytes + (tid % L::kWPerRow) * 16;
  }
  const uint8_t *ssrc = nullptr;
  if constexpr (WFMT == FMT_MXFP4) {
    const int srow = tid & (kTileW - 1);
    const int p = NPROJ == 2 ? srow / (kTileW / 2) : 0;
    const int frow = f0 + (NPROJ == 2 ? srow % (kTileW / 2) : srow);
    ssrc = a.s[p] + e * a.s_stride + (size_t)frow * (K / 32);
  }

  // one chunk's staged operands in registers
  struct Stage {
    glm_u32x4 x[L::kXPieces], w[L::kWPieces];
    uint32_t s;
  };
  auto load_stage = [&](int c, Stage &st) {
#pragma unroll
    for (int j = 0; j < L::kXPieces; ++j)
      st.x[j] = *reinterpret_cast<const glm_u32x4 *>(xsrc[j] + c * L::kChunk);
#pragma unroll
    for (int j = 0; j < L::kWPieces; ++j) st.w[j] = load_stream(wsrc[j] + c * L::kWRowBytes);
    st.s = 0;
    if constexpr (WFMT == FMT_MXFP4)
      if (tid < kTileW) st.s = *reinterpret_cast<const uint32_t *>(ssrc + c * (L::kChunk / 32));
  };
  auto store_stage = [&](int buf, const Stage &st) {
    uint8_t *base = smem + buf * L::kStageBytes;
    uint16_t *sx = reinterpret_cast<uint16_t *>(base);
    uint8_t *sw = base + L::kXBytes;
#pragma unroll
    for (int j = 0; j < L::kXPieces; ++j)
      *reinterpret_cast<glm_u32x4 *>(sx +
                                     (tid / L::kXPerRow + j * (kThreads / L::kXPerRow)) *
                                         L::kXStride +
                                     (tid % L::kXPerRow) * 8) = st.x[j];
#pragma unroll
    for (int j = 0; j < L::kWPieces; ++j)
      *reinterpret_cast<glm_u32x4 *>(sw +
                                     (tid / L::kWPerRow + j * (kThreads / L::kWPerRow)) *
                                         L::kWStride +
                                     (tid % L::kWPerRow) * 16) = st.w[j];
    if constexpr (WFMT == FMT_MXFP4) {
      uint32_t *ss = reinterpret_cast<uint32_t *>(sw + L::kWBytes);
      if (tid < kTileW) ss[tid] = st.s;
    }
  };

  glm_f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = glm_f32x4{0.f, 0.f, 0.f, 0.f};

  // this wave's 4 weight-row tiles within the 256 staged rows (gate/up: two
  // gate tiles, then the up tiles of the same features)
  auto wrow_of = [&](int rt) {
    return NPROJ == 2 ? (rt / 2) * (kTileW / 2) + wf * 32 + (rt % 2) * 16 : wf * 64 + rt * 16;
  };

  // MFMAs of one staged chunk
  auto compute = [&](int buf) {
    const uint8_t *base = smem + buf * L::kStageBytes;
    const uint16_t *sx = reinterpret_cast<const uint16_t *>(base);
    const uint8_t *sw = base + L::kXBytes;
    if constexpr (WFMT == FMT_MXFP4) {
      const uint32_t *ss = reinterpret_cast<const uint32_t *>(sw + L::kWBytes);
      glm_u32x4 raw[4];
      float scale[4];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const int wr = wrow_of(rt) + r;
        raw[rt] = *reinterpret_cast<const glm_u32x4 *>(sw + wr * L::kWStride + 16 * q);
        scale[rt] = e8m0_to_f32((ss[wr] >> (8 * q)) & 0xffu);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        glm_bf16x8 xb[4];
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          xb[ct] = *reinterpret_cast<const glm_bf16x8 *>(
              sx + (wt * 64 + ct * 16 + r) * L::kXStride + 32 * q + 8 * i);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          const glm_bf16x8 af = mxfp4_word_to_bf16x8(raw[rt][i], scale[rt]);
#pragma unroll
          for (int ct = 0; ct < 4; ++ct)
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, xb[ct], acc[rt][ct], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < L::kChunk / 32; ++i) {
        glm_bf16x8 xb[4], af[4];
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          xb[ct] = *reinterpret_cast<const glm_bf16x8 *>(
              sx + (wt * 64 + ct * 16 + r) * L::kXStride + 32 * i + 8 * q);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
          af[rt] = *reinterpret_cast<const glm_bf16x8 *>(sw + (wrow_of(rt) + r) * L::kWStride +
                                                         64 * i + 16 * q);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int ct = 0; ct < 4; ++ct)
            acc[rt][ct] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rt], xb[ct], acc[rt][ct], 0, 0, 0);
      }
    }
  };

  Stage st;
  load_stage(0, st);
  store_stage(0, st);
  __syncthreads();
  // steady state: next chunk's loads in flight during this chunk's MFMAs; the
  // last chunk is peeled so the loop body has no conditional work
  for (int c = 0; c + 1 < nchunks; ++c) {
    load_stage(c + 1, st);
    compute(c & 1);
    store_stage((c + 1) & 1, st);
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
      for (int i = 0; i < 2; ++i) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
          o[m] = f32_to_bf16(limited_swiglu(bf16_round(acc[i][ct][m]),
                                            bf16_round(acc[2 + i][ct][m]), a.limit));
        store_rows4(orow + f0 + wf * 32 + i * 16 + 4 * q, o);
      }
    } else {
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = f32_to_bf16(acc[rt][ct][m]);
        store_rows4(orow + f0 + wf * 64 + rt * 16 + 4 * q, o);
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
  return d % 128 == 0 && I % 128 == 0 && d % 256 == 0;
}

static int grouped_launch(hipStream_t stream, GroupedArgs a, int nproj, int wfmt, int max_tiles) {
  a.feature_tiles = a.N / (nproj == 2 ? kTileW / 2 : kTileW);
  // XCD x handles items [x * per, (x + 1) * per) with per <= ceil(max_items / 8),
  // at linear ids x + 8k: the grid must reach 8 * ceil(max_items / 8)
  const long long max_items = (long long)max_tiles * a.feature_tiles;
  const dim3 grid((unsigned)(((max_items + kXcds - 1) / kXcds) * kXcds));
  if (wfmt == FMT_MXFP4) {
    const size_t lds = 2 * (size_t)GroupedLayout<FMT_MXFP4>::kStageBytes;
    if (nproj == 2)
      hipLaunchKernelGGL((grouped_mx_gemm_kernel<2, FMT_MXFP4>), grid, dim3(kThreads), lds,
                         stream, a);
    else
      hipLaunchKernelGGL((grouped_mx_gemm_kernel<1, FMT_MXFP4>), grid, dim3(kThreads), lds,
                         stream, a);
  } else {
    const size_t lds = 2 * (size_t)GroupedLayout<FMT_BF16>::kStageBytes;
    if (nproj == 2)
      hipLaunchKernelGGL((grouped_mx_gemm_kernel<2, FMT_BF16>), grid, dim3(kThreads), lds,
                         stream, a);
    else
      hipLaunchKernelGGL((grouped_mx_gemm_kernel<1, FMT_BF16>), grid, dim3(kThreads), lds,
                         stream, a);
  }
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
  return grouped_launch(stream, a, 2, FMT_MXFP4, max_tiles);
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
  return grouped_launch(stream, a, 1, FMT_MXFP4, max_tiles);
}

// Dense bf16 SwiGLU MLP over T token rows (the shared expert at many tokens):
// h = limited_swiglu(bf16(x Wg^T), bf16(x Wu^T)); out = bf16(h Wd^T).
bool glm_grouped_dense_mlp_supported(int T, int d, int I, int fmt) {
  return fmt == FMT_BF16 && T >= 256 && d % 256 == 0 && I % 128 == 0;
}

int glm_grouped_dense_mlp_launch(hipStream_t stream, const uint16_t *x, int T, int d, int I,
                                 const uint16_t *gw, const uint16_t *uw, const uint16_t *dw,
                                 float limit, uint16_t *h, uint16_t *out) {
  const int tiles = (T + kTileM - 1) / kTileM;
  GroupedArgs a{};
  a.act = x;
  a.dense_rows = T;
  a.w[0] = reinterpret_cast<const uint8_t *>(gw);
  a.w[1] = reinterpret_cast<const uint8_t *>(uw);
  a.N = I;
  a.K = d;
  a.out = h;
  a.limit = glm_limit_bf16(limit);
  int rc = grouped_launch(stream, a, 2, FMT_BF16, tiles);
  if (rc) return rc;
  GroupedArgs b{};
  b.act = h;
  b.dense_rows = T;
  b.w[0] = b.w[1] = reinterpret_cast<const uint8_t *>(dw);
  b.N = d;
  b.K = I;
  b.out = out;
  return grouped_launch(stream, b, 1, FMT_BF16, tiles);
}

bool glm_grouped_supported(int d, int I);

extern "C" int glm_expert_gate_up_grouped(void *stream, const uint16_t *x, int d, int I,
                                          const uint8_t *gate_packed, const uint8_t *gate_scales,
                                          const uint8_t *up_packed, const uint8_t *up_scales,
                                          const int32_t *pair_token, const int32_t *tiles,
                                          const int32_t *num_tiles, int max_tiles,
                                          float swiglu_limit, uint16_t *h) {
  glm::clear_error();
  GLM_REQUIRE(x && gate_packed && gate_scales && up_packed && up_scales && pair_token && tiles &&
                  num_tiles && h,
              GLM_ERR_INVALID_ARGUMENT, "expert_gate_up_grouped: null pointer argument");
  GLM_REQUIRE(max_tiles >= 0, GLM_ERR_INVALID_ARGUMENT, "expert_gate_up_grouped: max_tiles < 0");
  GLM_REQUIRE(glm_grouped_supported(d, I), GLM_ERR_UNSUPPORTED_SHAPE,
              "expert_gate_up_grouped: needs d %% 256 == 0 and I %% 128 == 0 (d=%d I=%d)", d, I);
  GLM_REQUIRE(glm_aligned16({x, gate_packed, up_packed, tiles, h}), GLM_ERR_INVALID_ARGUMENT,
              "expert_gate_up_grouped: buffers must be 16-byte aligned");
  if (max_tiles == 0) return GLM_OK;
  return glm_grouped_gate_up_launch((hipStream_t)stream, x, pair_token,
                                    reinterpret_cast<const int4 *>(tiles), num_tiles, max_tiles,
                                    d, I, gate_packed, gate_scales, up_packed, up_scales, h,
                                    swiglu_limit);
}

extern "C" int glm_expert_down_grouped(void *stream, const uint16_t *h, int I, int d,
                                       const uint8_t *down_packed, const uint8_t *down_scales,
                                       const int32_t *tiles, const int32_t *num_tiles,
                                       int max_tiles, uint16_t *y) {
  glm::clear_error();
  GLM_REQUIRE(h && down_packed && down_scales && tiles && num_tiles && y,
              GLM_ERR_INVALID_ARGUMENT, "expert_down_grouped: null pointer argument");
  GLM_REQUIRE(max_tiles >= 0, GLM_ERR_INVALID_ARGUMENT, "expert_down_grouped: max_tiles < 0");
  GLM_REQUIRE(glm_grouped_supported(d, I), GLM_ERR_UNSUPPORTED_SHAPE,
              "expert_down_grouped: needs d %% 256 == 0 and I %% 128 == 0 (d=%d I=%d)", d, I);
  GLM_REQUIRE(glm_aligned16({h, down_packed, tiles, y}), GLM_ERR_INVALID_ARGUMENT,
              "expert_down_grouped: buffers must be 16-byte aligned");
  if (max_tiles == 0) return GLM_OK;
  return glm_grouped_down_launch((hipStream_t)stream, h, reinterpret_cast<const int4 *>(tiles),
                                 num_tiles, max_tiles, I, d, down_packed, down_scales, y);
}
