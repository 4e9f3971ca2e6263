// Prefill grouped GEMMs of the routed experts (and the dense shared expert)
// on gfx950 MFMA.
//
// For every routed expert e with n_e > 0 rows in dispatch (sorted) order
// (native_expert_ssd.py:726-743 runs gather_qmm over all (t, j) pairs):
//   gate/up: h[pos] = limited_swiglu(bf16(x[tok(pos)] . Wg_e^T), bf16(x[tok(pos)] . Wu_e^T))
//   down:    y[pos] = bf16(h[pos] . Wd_e^T)
// and, in dense mode (one "expert", rows = tokens), the bf16 shared expert
// DenseMLP (layers.py:160-171) at many tokens.  The routed MXFP4 experts run
// on the block-scaled GEMMs further down; the bf16 kernel here serves the
// dense shared expert.
//
// The dispatch cuts each routed expert's rows into row tiles of at most 160
// rows (the block-scaled GEMMs below); the dense bf16 kernel cuts the tokens
// into tiles of kTileM = 128 rows.  A workgroup of the bf16 kernel computes
// one row tile against kTileW = 256 weight rows (gate/up: 128 features of each
// projection; down: 256 features) in a 4 x 2 arrangement of eight waves: wave
// (wf, wt) owns 64 weight rows x 64 tokens, i.e. 4 x 4 accumulator tiles of
// v_mfma_f32_16x16x32_bf16 (two waves per SIMD, so one wave's LDS reads
// overlap the other's MFMAs).  Gate/up grids that would stay below one
// workgroup per CU take 192-row tiles instead (2 x 4 waves of 96 rows x 32
// tokens).  K advances in chunks of 64: the activation rows
// and the weight rows of a chunk are staged in LDS, three stages deep, and the
// next chunks' global loads are issued before the current chunk's MFMAs.
// MFMA i, slot s of lane (r, q) is K = 32i + 8q + s.
//
// Workgroup -> (row tile, feature tile) is XCD-aware: workgroups are dealt to
// the 8 XCDs round-robin by linear id, so XCD x takes the x-th contiguous
// eighth of the work items, ordered row tile major.  The feature tiles of one
// row tile (which share its activation rows) and the row tiles of one expert
// (which share its weights) then run side by side on one XCD and meet in its
// L2.  Items past the real tile count (known only on the device) exit.
#include "lds_stage.h"
#include "mfma_tile.h"

namespace glm {

constexpr int kTileM = 128;    // token rows per tile
constexpr int kTileW = 256;    // weight rows per workgroup
constexpr int kThreads = 512;  // 8 waves: 4 along the weight rows x 2 along the tokens
constexpr int kWaves = kThreads / 64;
constexpr int kXcds = 8;
constexpr int kNumCUs = 256;  // MI355X
constexpr int kStages = 3;     // LDS ring: two chunks in flight while one is consumed

// One K chunk of a workgroup's operands in LDS, unpadded and XOR-swizzled in
// 16-byte pieces so that the MFMA operand reads (16 rows x one piece column)
// hit distinct banks:
//   activations  [kTileM rows][kChunk bf16]   piece p of row R at p ^ xswz(R)
//   weights      [kTileW rows][kWRowBytes]    piece p of row R at p ^ wswz(R)
//   scales       [kTileW rows] u32            (MXFP4: the chunk's 4 E8M0 bytes)
// Direct global->LDS loads write one wave's 64 x 16 bytes contiguously, so a
// lane's LDS slot is fixed by its lane id; each lane fetches the global piece
// that belongs in its slot.
template <int TW>
struct Bf16Layout {
  static constexpr int kChunk = 64;  // K per stage
  static constexpr int kXRowBytes = kChunk * 2;
  static constexpr int kWRowBytes = kChunk * 2;
  static constexpr int kXBytes = kTileM * kXRowBytes;
  static constexpr int kWBytes = TW * kWRowBytes;
  static constexpr int kStageBytes = kXBytes + kWBytes;
  static constexpr int kXPerRow = kXRowBytes / 16;  // pieces per row
  static constexpr int kWPerRow = kWRowBytes / 16;
  static constexpr int kXLoads = kXBytes / (kThreads * 16);  // 16-byte loads per thread
  static constexpr int kWLoads = kWBytes / (kThreads * 16);
  static constexpr int kLoads = kXLoads + kWLoads;  // per chunk, per thread
  static_assert(kXBytes % (kThreads * 16) == 0 && kWBytes % (kThreads * 16) == 0, "staging");
  static_assert(kStages * kStageBytes <= 160 * 1024, "LDS ring exceeds 160 KB");
  static_assert(kWaves * 16 * 144 <= kStageBytes, "the down epilogue's staging fits a stage");

  // 128-byte rows of 8 pieces: swizzle over the row's low 3 bits
  __device__ static int xswz(int row) { return row & 7; }
  __device__ static int wswz(int row) { return row & 7; }
};

struct GroupedArgs {
  const uint16_t *act;       // gate/up: x [T][K]; down: h [T][K]
  int dense_rows;            // T: tiles of kTileM consecutive rows
  const uint8_t *w[2];       // bf16 weights [N][K] per projection
  int N, K;                  // weight rows per expert and projection; reduction length
  int feature_tiles;         // workgroups along N per row tile
  uint16_t *out;             // bf16 [rows][N]
  float limit;               // bf16-rounded SwiGLU limit (gate/up)
};

// Direct global->LDS loads: lane i's 16 bytes land at lds + 16 i;
// the LDS address is wave-uniform.
__device__ __forceinline__ void load16_to_lds(const void *src, void *lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}

// Wave arrangement of a TW-row weight tile: WF waves along the weight rows x
// WT along the tokens, each wave BR x BT MFMA blocks of 16 x 16.  TW = 256:
// 4 x 2 waves of 64 rows x 64 tokens; TW = 192 (gate/up: 96 features of each
// projection, for grids that 256-row tiles leave below one workgroup per CU):
// 2 x 4 waves of 96 rows x 32 tokens.
template <int TW>
struct Bf16Waves {
  static constexpr int WF = TW == 256 ? 4 : 2;
  static constexpr int WT = kWaves / WF;
  static constexpr int BR = TW / (16 * WF);
  static constexpr int BT = kTileM / (16 * WT);
  static_assert(WF * BR * 16 == TW && WT * BT * 16 == kTileM, "wave tiles cover the tile");
};

// One workgroup's work item of the bf16 GEMM; lin is its index in the
// launch's range of these workgroups (a multiple of kXcds covering every item).
template <int NPROJ, int TW>
__device__ __forceinline__ void bf16_gemm_item(const GroupedArgs &a, int lin) {
  using L = Bf16Layout<TW>;
  using WV = Bf16Waves<TW>;
  static_assert(NPROJ == 2 || TW == 256, "192-row tiles pair gate and up");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nft = a.feature_tiles;
  const int ntiles = (a.dense_rows + kTileM - 1) / kTileM;
  const int items = ntiles * nft;
  const int per_xcd = (items + kXcds - 1) / kXcds;
  const int k_on_xcd = lin / kXcds;
  const int item = (lin % kXcds) * per_xcd + k_on_xcd;
  if (k_on_xcd >= per_xcd || item >= items) return;
  const int tile_id = item / nft, ftile = item % nft;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int wf = wave % WV::WF, wt = wave / WV::WF;
  const int pos0 = tile_id * kTileM, rows = min(kTileM, a.dense_rows - pos0);
  const int K = a.K;
  const int nchunks = K / L::kChunk;
  // weight rows of this workgroup: NPROJ == 2 -> [gate f0..f0+TW/2 | up f0..f0+TW/2]
  const int f0 = ftile * (TW / NPROJ);
  const int wrow_bytes = K * 2;

  // ---- load assignment (fixed over the K loop).  Load j of wave w fills the
  // (j * kWaves + w)-th 1 KB block of the stage region.
  const uint8_t *xsrc[L::kXLoads];
#pragma unroll
  for (int j = 0; j < L::kXLoads; ++j) {
    const int slot = (j * kWaves + wave) * 64 + lane;  // 16-byte slot in the region
    const int row = slot / L::kXPerRow, piece = (slot % L::kXPerRow) ^ L::xswz(row);
    // rows past the tile's end re-read its first row: MFMA columns are
    // independent and those columns are never stored
    const int pos = pos0 + (row < rows ? row : 0);
    const long long arow = pos;
    xsrc[j] = reinterpret_cast<const uint8_t *>(a.act + arow * K) + piece * 16;
  }
  const uint8_t *wsrc[L::kWLoads];
#pragma unroll
  for (int j = 0; j < L::kWLoads; ++j) {
    const int slot = (j * kWaves + wave) * 64 + lane;
    const int row = slot / L::kWPerRow, piece = (slot % L::kWPerRow) ^ L::wswz(row);
    // (a select, not a.w[p]: a lane-varying index into the kernel arguments
    // becomes a vector memory load)
    const uint8_t *wbase = NPROJ == 2 && row >= TW / 2 ? a.w[1] : a.w[0];
    const int frow = f0 + (NPROJ == 2 ? row % (TW / 2) : row);
    wsrc[j] = wbase + (size_t)frow * wrow_bytes + piece * 16;
  }

  // Direct global->LDS loads of chunk c into ring stage `stage`.
  auto issue = [&](int c, int stage) {
    uint8_t *base = smem + stage * L::kStageBytes;
#pragma unroll
    for (int j = 0; j < L::kXLoads; ++j)
      load16_to_lds(xsrc[j] + c * L::kXRowBytes, base + (j * kWaves + wave) * 1024);
#pragma unroll
    for (int j = 0; j < L::kWLoads; ++j)
      load16_to_lds(wsrc[j] + c * L::kWRowBytes, base + L::kXBytes + (j * kWaves + wave) * 1024);
  };

  constexpr int BR = WV::BR, BT = WV::BT, HB = BR / 2;
  glm_f32x4 acc[BR][BT];
#pragma unroll
  for (int i = 0; i < BR; ++i)
#pragma unroll
    for (int j = 0; j < BT; ++j) acc[i][j] = glm_f32x4{0.f, 0.f, 0.f, 0.f};

  // this wave's BR weight-row tiles within the TW staged rows (gate/up: HB
  // gate tiles, then the up tiles of the same features)
  auto wrow_of = [&](int rt) {
    return NPROJ == 2 ? (rt / HB) * (TW / 2) + wf * HB * 16 + (rt % HB) * 16 : wf * BR * 16 + rt * 16;
  };
  // MFMAs of one staged chunk: MFMA i, slot s of lane (r, q) is K = 32i + 8q + s.
  auto compute = [&](int stage) {
    const uint8_t *base = smem + stage * L::kStageBytes;
    const uint8_t *sx = base;
    const uint8_t *sw = base + L::kXBytes;
    {
#pragma unroll
      for (int i = 0; i < L::kChunk / 32; ++i) {
        glm_bf16x8 xb[BT], af[BR];
#pragma unroll
        for (int ct = 0; ct < BT; ++ct) {
          const int xr = wt * BT * 16 + ct * 16 + r;
          xb[ct] = *reinterpret_cast<const glm_bf16x8 *>(sx + xr * L::kXRowBytes +
                                                         16 * ((4 * i + q) ^ L::xswz(xr)));
        }
#pragma unroll
        for (int rt = 0; rt < BR; ++rt) {
          const int wr = wrow_of(rt) + r;
          af[rt] = *reinterpret_cast<const glm_bf16x8 *>(sw + wr * L::kWRowBytes +
                                                         16 * ((4 * i + q) ^ L::wswz(wr)));
        }
#pragma unroll
        for (int rt = 0; rt < BR; ++rt)
#pragma unroll
          for (int ct = 0; ct < BT; ++ct)
            acc[rt][ct] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rt], xb[ct], acc[rt][ct], 0, 0, 0);
      }
    }
  };

  // Ring: chunks c + 1 and c + 2 are in flight while chunk c is consumed.  The
  // barrier of iteration c also guarantees that every wave has finished
  // chunk c - 1, whose stage the loads of chunk c + 2 overwrite.
  issue(0, 0);
  if (nchunks > 1) issue(1, 1);
  for (int c = 0; c < nchunks; ++c) {
    if (c + 1 < nchunks)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(L::kLoads));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    ring_barrier();
    if (c + 2 < nchunks) issue(c + 2, (c + 2) % kStages);
    compute(c % kStages);
  }

  // ---- epilogue: lane (r, q) of tile (rt, ct) holds features 4q..4q+3 of the
  // row tile for token column r
  if constexpr (NPROJ == 2) {
    // SwiGLU on pairs of elements (limited_swiglu2_fast: the hardware exp2 /
    // reciprocal sigmoid, one packed convert per bf16 rounding of a pair)
    const float lim = a.limit > 0.0f ? a.limit : __builtin_inff();
#pragma unroll
    for (int ct = 0; ct < BT; ++ct) {
      const int row = wt * BT * 16 + ct * 16 + r;
      if (row >= rows) continue;
      uint16_t *orow = a.out + (size_t)(pos0 + row) * a.N;
#pragma unroll
      for (int i = 0; i < HB; ++i) {
        float h[4];
#pragma unroll
        for (int m = 0; m < 4; m += 2) {
          float g0 = acc[i][ct][m], g1 = acc[i][ct][m + 1];
          float u0 = acc[HB + i][ct][m], u1 = acc[HB + i][ct][m + 1];
          bf16_round2(g0, g1);
          bf16_round2(u0, u1);
          limited_swiglu2_fast(g0, g1, u0, u1, lim, h[m], h[m + 1]);
        }
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = __float_as_uint(h[m]) >> 16;  // bf16-exact
        store_rows4(orow + f0 + wf * HB * 16 + i * 16 + 4 * q, o);
      }
    }
  } else {
    // the output through LDS, so that every store writes whole 128-byte
    // lines: per token block the wave's 16 rows x 64 features go to its own
    // 16 x 144 B area of the stage no chunk occupies (the ring's last loads
    // went to the other two) and come back 16 contiguous bytes per lane
    uint8_t *yst = smem + (nchunks % kStages) * L::kStageBytes + wave * (16 * 144);
    const int rr = lane >> 3, seg = lane & 7;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      if (wt * 64 + ct * 16 >= rows) continue;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = f32_to_bf16(acc[rt][ct][m]);
        *reinterpret_cast<uint2 *>(yst + r * 144 + (rt * 16 + 4 * q) * 2) =
            uint2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = wt * 64 + ct * 16 + 8 * h + rr;
        const glm_u32x4 v = *reinterpret_cast<const glm_u32x4 *>(yst + (8 * h + rr) * 144 + 16 * seg);
        if (row < rows)
          *reinterpret_cast<glm_u32x4 *>(a.out + (size_t)(pos0 + row) * a.N + f0 + wf * 64 + 8 * seg) = v;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

template <int NPROJ, int TW>
__global__ __launch_bounds__(kThreads) void grouped_bf16_gemm_kernel(GroupedArgs a) {
  bf16_gemm_item<NPROJ, TW>(a, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Routed expert GEMMs on the block-scaled MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4): MXFP4 weights enter as they are stored
// (E2M1 codes + their E8M0 group scales), the bf16 activations as a
// block-scaled split (32-element groups, E8M0 scales) in one of three forms:
//   ACT_FP8X2  x = hi * 2^(shi - 127) + lo * 2^(slo - 127), hi and lo E4M3FN.
//              hi holds the top 4 significant bits of each element, lo the
//              remaining <= 4 (a bf16 element has 8), so the split reproduces
//              every element exactly unless it lies ~14 binades below its
//              group's maximum, where the error stays below 2^-22 of that
//              maximum.  Two MFMAs per output block at the FP8 rate.
//   ACT_FP6X2  the same two-term form with E2M3 codes: ~3e-4 relative error
//              on Gaussian rows, two MFMAs at the FP6 rate (twice FP8's).
//   ACT_FP4    one E2M1 term: ~12 % relative error, one MFMA at the FP4 rate.
//   ACT_FP8FP6 hi E4M3FN (FP8 rate) + lo E2M3 (FP6 rate): exact for elements
//              at most two binades below their group maximum's; lo's
//              two-bit exponent bounds the error by max / 840, as ACT_FP6X2's.
// Each term's scale is the smallest power of two that keeps the group's
// largest magnitude within the element format's maximum (448, 7.5, 6); lo
// encodes the exact f32 residual x - hi.  The MFMAs accumulate in f32: no
// dequantisation instructions at all.
//
// Operand layout of the 16x16x128 MFMA, lane (i = l % 16, g = l / 16):
//   A = weights (E2M1, 16 bytes): weight row i, K [32g, 32g + 32) -- exactly
//       one stored MXFP4 group, so lane g's 16 bytes come straight from the
//       row and its scale operand is that group's E8M0 byte;
//   B = activations, token i: E4M3 (32 bytes) K [16g, 16g + 16) in bytes
//       0..15 and K [64 + 16g, 64 + 16g + 16) in bytes 16..31; E2M3 (24
//       bytes) and E2M1 (16 bytes) K [32g, 32g + 32), element s at bits
//       [w s, w s + w) of the lane's registers; scale operand: token i's E8M0
//       byte of group g (K [32g, 32g + 32));
//   D: lane holds weight rows 4g..4g+3 of token column i.
// ---------------------------------------------------------------------------

// Activation formats of the block-scaled GEMMs (the C ABI's act_format).
constexpr int ACT_FP8X2 = 0, ACT_FP6X2 = 1, ACT_FP4 = 2, ACT_FP8FP6 = 3;

__host__ __device__ constexpr int act_terms(int af) { return af == ACT_FP4 ? 1 : 2; }
// Stored code bytes of one term per activation row of K elements.
__host__ __device__ constexpr long long act_code_row(int K, int af) {
  return af == ACT_FP4 ? K / 2 : K;
}

// Byte offsets of an activation split of `rows` x K: hi codes, lo codes,
// hi scales, lo scales, each 256-byte aligned (ACT_FP4: codes, scales).
// Code rows: ACT_FP8X2 one byte per element; ACT_FP4 two per byte, low
// nibble first (the MXFP4 weight layout); ACT_FP6X2 per 128-element chunk
// 128 bytes: group g's 32 codes packed 6 bits each, low bits first, bytes
// 0..15 at 16 g and bytes 16..23 at 64 + 16 g (so that the FP8 operand reads
// -- 16 bytes at 16 g and at 64 + 16 g -- fetch a whole E2M3 operand; the
// other 8 bytes are zero).
struct SplitLayout {
  size_t lo, shi, slo, total;
  __host__ __device__ SplitLayout(long long rows, int K, int af = ACT_FP8X2) {
    const size_t codes = ((size_t)(rows * act_code_row(K, af)) + 255) & ~(size_t)255;
    const size_t scales = ((size_t)rows * (K / 32) + 255) & ~(size_t)255;
    const int n = act_terms(af);
    lo = codes;
    shi = n * codes;
    slo = shi + scales;  // ACT_FP4: past the end, unused
    total = n * (codes + scales);
  }
};

// E8M0 exponent byte for a group whose largest magnitude is amax: the
// smallest 2^(b - 127) with amax / 2^(b - 127) <= mmax 2^emax, the element
// format's maximum (mmax in [0.5, 1)); 127 for an all-zero group.
__device__ __forceinline__ int fit_scale_byte(float amax, float mmax, int emax) {
  if (!(amax > 0.0f)) return 127;
  int e;
  const float m = frexpf(amax, &e);  // amax = m 2^e, m in [0.5, 1)
  const int k = m <= mmax ? e - emax : e - emax + 1;
  return min(max(k + 127, 0), 254);
}
// E4M3FN: maximum 448 = 0.875 2^9
__device__ __forceinline__ int split_scale_byte(float amax) { return fit_scale_byte(amax, 0.875f, 9); }

// Four lanes per 32-element group, eight elements each: hi/lo E4M3FN codes and
// their scales.  A wave loads 1 KB of contiguous bf16 per instruction and
// stores 512 contiguous bytes of codes; the group maxima are combined over the
// lane quad with DPP.  (One lane per group loaded 64 B strides per instruction.)
__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, true)));
  return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, true)));
}
// The FP8 hi/lo split of one 32-element scale group held 8 per lane by four
// lanes: v holds this lane's elements (hi and lo codes of v[4 j .. 4 j + 3] go
// to ch[j] / cl[j]); gmax(a) is the maximum of a over the group's four lanes.
// The scaled converts divide by (down) and multiply by (up) the f32 scale
// operand, of which only the exponent field counts: the E8M0 byte b shifted
// into that field stands for 2^(b - 127), also for b = 0.  Codes and residuals
// are those of ldexp by 127 - b and the unscaled converts (checked on the
// device for every byte class, FP8 subnormals and ties).
template <typename GroupMax>
__device__ __forceinline__ void fp8_split_lane8(float v[8], GroupMax gmax, uint32_t ch[2],
                                                uint32_t cl[2], int &bh, int &bl) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
  bh = split_scale_byte(gmax(amax));
  const float sh = __uint_as_float((uint32_t)bh << 23);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    s16x2 w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(s16x2{0, 0}, v[4 * j], v[4 * j + 1], sh, false);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, v[4 * j + 2], v[4 * j + 3], sh, true);
    ch[j] = __builtin_bit_cast(uint32_t, w);
    // residuals, exact in f32
    v[4 * j] -= __builtin_amdgcn_cvt_scalef32_f32_fp8(ch[j], sh, 0);
    v[4 * j + 1] -= __builtin_amdgcn_cvt_scalef32_f32_fp8(ch[j], sh, 1);
    v[4 * j + 2] -= __builtin_amdgcn_cvt_scalef32_f32_fp8(ch[j], sh, 2);
    v[4 * j + 3] -= __builtin_amdgcn_cvt_scalef32_f32_fp8(ch[j], sh, 3);
  }
  float ramax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ramax = fmaxf(ramax, fabsf(v[j]));
  bl = split_scale_byte(gmax(ramax));
  const float sl = __uint_as_float((uint32_t)bl << 23);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    s16x2 w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(s16x2{0, 0}, v[4 * j], v[4 * j + 1], sl, false);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, v[4 * j + 2], v[4 * j + 3], sl, true);
    cl[j] = __builtin_bit_cast(uint32_t, w);
  }
}

__device__ __forceinline__ void act_split_one(const uint16_t *x, long long groups, long long i,
                                              uint8_t *hi, uint8_t *lo, uint8_t *shi,
                                              uint8_t *slo) {
  const long long g = i >> 2;
  const int part = (int)(i & 3);  // elements 8 part .. 8 part + 7 of the group
  if (g >= groups) return;        // whole lane quads leave together
  const glm_u32x4 w = *reinterpret_cast<const glm_u32x4 *>(x + g * 32 + 8 * part);
  float v[8];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    v[2 * h] = __uint_as_float(w[h] << 16);
    v[2 * h + 1] = __uint_as_float(w[h] & 0xffff0000u);
  }
  uint32_t ch[2], cl[2];
  int bh, bl;
  fp8_split_lane8(v, [](float m) { return quad_max(m); }, ch, cl, bh, bl);
  *reinterpret_cast<uint2 *>(hi + g * 32 + 8 * part) = uint2{ch[0], ch[1]};
  *reinterpret_cast<uint2 *>(lo + g * 32 + 8 * part) = uint2{cl[0], cl[1]};
  if (part == 0) {
    shi[g] = (uint8_t)bh;
    slo[g] = (uint8_t)bl;
  }
}

__global__ __launch_bounds__(256) void act_split_kernel(const uint16_t *x, long long groups,
                                                        uint8_t *hi, uint8_t *lo, uint8_t *shi,
                                                        uint8_t *slo) {
  act_split_one(x, groups, (long long)blockIdx.x * blockDim.x + threadIdx.x, hi, lo, shi, slo);
}

// The prefill layer's two splits in one launch: blocks [0, wblocks) split the
// router weights into three bf16 parts (as router_weight_split_kernel), the
// rest form x's FP8 hi/lo split (as act_split_kernel).
__global__ __launch_bounds__(256) void prefill_split_kernel(const float *rw, long long nw,
                                                            uint16_t *ws, int wblocks,
                                                            const uint16_t *x, long long groups,
                                                            uint8_t *hi, uint8_t *lo,
                                                            uint8_t *shi, uint8_t *slo) {
  if ((int)blockIdx.x < wblocks) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nw) bf16x3_split_one(rw, nw, ws, i);
    return;
  }
  act_split_one(x, groups, (long long)(blockIdx.x - wblocks) * blockDim.x + threadIdx.x, hi, lo,
                shi, slo);
}

// E2M3 / E2M1 code of v 2^(127 - b), round to nearest even, saturating at the
// format maximum; *back = the code's value times 2^(b - 127) (exact in f32).
// E2M3 magnitudes are n / 8 below 2, n / 4 in [2, 4), n / 2 in [4, 7.5]
// (codes n, n + 8, n + 16); E2M1's are n / 2, n, 2 n (codes n, n + 2, n + 4).
template <int AF>
__device__ __forceinline__ uint32_t lowp_code(float v, int b, float *back) {
  constexpr float kMax = AF == ACT_FP6X2 ? 7.5f : 6.0f;
  constexpr int kFrac = AF == ACT_FP6X2 ? 3 : 1;  // log2 of the quantum's inverse below 2
  constexpr uint32_t kSign = AF == ACT_FP6X2 ? 0x20u : 0x8u;
  const float y = fminf(ldexpf(fabsf(v), 127 - b), kMax);
  const int e = y < 2.0f ? 0 : (y < 4.0f ? 1 : 2);
  const float n = rintf(ldexpf(y, kFrac - e));
  const uint32_t neg = __float_as_uint(v) >> 31;
  const float mag = ldexpf(n, e - kFrac + b - 127);
  *back = neg ? -mag : mag;
  return ((uint32_t)n + (uint32_t)(e << kFrac)) | (neg ? kSign : 0u);
}

// Codes of one term of a group: E2M3 six bits each into 6 words, E2M1 four
// bits into 4 words, element s at bits [w s, w s + w).
template <int AF>
__device__ __forceinline__ void lowp_term(float v[32], int b, uint32_t out[6]) {
  constexpr int w = AF == ACT_FP6X2 ? 6 : 4;
#pragma unroll
  for (int j = 0; j < 6; ++j) out[j] = 0u;
#pragma unroll
  for (int s = 0; s < 32; ++s) {
    float back;
    const uint32_t c = lowp_code<AF>(v[s], b, &back);
    v[s] -= back;  // the exact residual
    const int pos = w * s;
    out[pos >> 5] |= c << (pos & 31);
    if ((pos & 31) + w > 32) out[(pos >> 5) + 1] |= c >> (32 - (pos & 31));
  }
}

// One thread per 32-element group: the ACT_FP8FP6 split -- hi E4M3FN codes
// and scale exactly as act_split_kernel forms them, lo the E2M3 code of the
// exact residual in the ACT_FP6X2 layout.
__global__ __launch_bounds__(256) void act_split_fp8fp6_kernel(const uint16_t *x, long long groups,
                                                               int K, uint8_t *hi, uint8_t *lo,
                                                               uint8_t *shi, uint8_t *slo) {
  const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  const glm_u32x4 *src = reinterpret_cast<const glm_u32x4 *>(x + g * 32);
  float v[32];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const glm_u32x4 w = src[j];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      v[8 * j + 2 * h] = __uint_as_float(w[h] << 16);
      v[8 * j + 2 * h + 1] = __uint_as_float(w[h] & 0xffff0000u);
    }
  }
  const long long row = g / (K / 32);
  const int grp = (int)(g % (K / 32));
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
  const int bh = split_scale_byte(amax);
  uint32_t ch[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    int c = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(v[4 * j], 127 - bh),
                                            ldexpf(v[4 * j + 1], 127 - bh), 0, false);
    c = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(v[4 * j + 2], 127 - bh),
                                        ldexpf(v[4 * j + 3], 127 - bh), c, true);
    ch[j] = (uint32_t)c;
    v[4 * j] -= ldexpf(__builtin_amdgcn_cvt_f32_fp8(c, 0), bh - 127);
    v[4 * j + 1] -= ldexpf(__builtin_amdgcn_cvt_f32_fp8(c, 1), bh - 127);
    v[4 * j + 2] -= ldexpf(__builtin_amdgcn_cvt_f32_fp8(c, 2), bh - 127);
    v[4 * j + 3] -= ldexpf(__builtin_amdgcn_cvt_f32_fp8(c, 3), bh - 127);
  }
  float ramax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) ramax = fmaxf(ramax, fabsf(v[j]));
  const int bl = fit_scale_byte(ramax, 0.9375f, 3);  // E2M3: 7.5 = 0.9375 2^3
  uint32_t cl[6];
  lowp_term<ACT_FP6X2>(v, bl, cl);
  uint8_t *dh = hi + row * K + 32 * grp;
  *reinterpret_cast<glm_u32x4 *>(dh) = glm_u32x4{ch[0], ch[1], ch[2], ch[3]};
  *reinterpret_cast<glm_u32x4 *>(dh + 16) = glm_u32x4{ch[4], ch[5], ch[6], ch[7]};
  uint8_t *dl = lo + row * K + 128 * (grp >> 2) + 16 * (grp & 3);
  *reinterpret_cast<glm_u32x4 *>(dl) = glm_u32x4{cl[0], cl[1], cl[2], cl[3]};
  *reinterpret_cast<glm_u32x4 *>(dl + 64) = glm_u32x4{cl[4], cl[5], 0u, 0u};
  shi[g] = (uint8_t)bh;
  slo[g] = (uint8_t)bl;
}

// One thread per 32-element group: the ACT_FP6X2 (hi, lo) or ACT_FP4 split.
template <int AF>
__global__ __launch_bounds__(256) void act_split_lowp_kernel(const uint16_t *x, long long groups,
                                                             int K, uint8_t *hi, uint8_t *lo,
                                                             uint8_t *shi, uint8_t *slo) {
  constexpr float kMm = AF == ACT_FP6X2 ? 0.9375f : 0.75f;  // 7.5 = 0.9375 2^3, 6 = 0.75 2^3
  const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  const glm_u32x4 *src = reinterpret_cast<const glm_u32x4 *>(x + g * 32);
  float v[32];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const glm_u32x4 w = src[j];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      v[8 * j + 2 * h] = __uint_as_float(w[h] << 16);
      v[8 * j + 2 * h + 1] = __uint_as_float(w[h] & 0xffff0000u);
    }
  }
  const long long groups_per_row = K / 32;
  const long long row = g / groups_per_row;
  const int grp = (int)(g % groups_per_row);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
  const int bh = fit_scale_byte(amax, kMm, 3);
  uint32_t c[6];
  lowp_term<AF>(v, bh, c);
  shi[g] = (uint8_t)bh;
  if constexpr (AF == ACT_FP4) {
    *reinterpret_cast<glm_u32x4 *>(hi + row * (K / 2) + 16 * grp) = glm_u32x4{c[0], c[1], c[2], c[3]};
  } else {
    uint8_t *dh = hi + row * K + 128 * (grp >> 2) + 16 * (grp & 3);
    *reinterpret_cast<glm_u32x4 *>(dh) = glm_u32x4{c[0], c[1], c[2], c[3]};
    *reinterpret_cast<glm_u32x4 *>(dh + 64) = glm_u32x4{c[4], c[5], 0u, 0u};
    float ramax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) ramax = fmaxf(ramax, fabsf(v[j]));
    const int bl = fit_scale_byte(ramax, kMm, 3);
    lowp_term<AF>(v, bl, c);
    uint8_t *dl = lo + row * K + 128 * (grp >> 2) + 16 * (grp & 3);
    *reinterpret_cast<glm_u32x4 *>(dl) = glm_u32x4{c[0], c[1], c[2], c[3]};
    *reinterpret_cast<glm_u32x4 *>(dl + 64) = glm_u32x4{c[4], c[5], 0u, 0u};
    slo[g] = (uint8_t)bl;
  }
}

// Maximum over the four lanes l, l ^ 16, l ^ 32, l ^ 48: gfx950's row swaps
// (one VALU instruction each, no LDS round trip).
__device__ __forceinline__ float quad_row_max(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}

// The split of one 32-element scale group held 8 per lane by the four lanes
// q = 0..3 of a lane row (lanes r, r + 16, r + 32, r + 48); v holds this
// lane's elements 16 i + 4 q + m at v[4 i + m].  The arithmetic of
// act_split_kernel: ch[i] / cl[i] are the hi / lo codes of elements
// 16 i + 4 q .. + 3, bh / bl the group's scale bytes.
__device__ __forceinline__ void split_group_part(float v[8], uint32_t ch[2], uint32_t cl[2],
                                                 int *bh_out, int *bl_out) {
  fp8_split_lane8(v, [](float m) { return quad_row_max(m); }, ch, cl, *bh_out, *bl_out);
}

struct SplitArgs {
  const uint8_t *xhi, *xlo;    // activation codes (SplitLayout)
  const uint8_t *xshi, *xslo;  // activation scales [rows][K/32]
  uint32_t split_bytes;        // the split buffer starting at xhi (SplitLayout)
  const int32_t *act_index;    // sorted position -> activation row (nullptr: the position)
  const int4 *tiles;           // {expert, first sorted position, rows, 0}
  const int32_t *num_tiles;    // device-side count, read once and clamped to max_tiles
  int max_tiles;               // entries of `tiles` (the grid is sized for them)
  const uint8_t *w[2];         // stacked MXFP4 weights [E][N][K/2] per projection
  const uint8_t *s[2];         // stacked E8M0 scales [E][N][K/32]
  long long w_stride, s_stride;
  int N, K;
  int feature_tiles;
  uint16_t *out;               // bf16 [rows][N]
  float limit;
  // gate/up, ACT_FP8X2: when set, the epilogue writes the FP8 hi/lo split of
  // h (the down GEMM's input, SplitLayout(out_rows, N)) instead of h itself
  uint8_t *out_split;
  long long out_rows;
};

// Workgroup tile of the block-scaled GEMMs: up to 160 token rows (a row tile
// of the dispatch) x 512 weight rows (gate/up: 256 features of each
// projection), 16 waves as 8 (weight rows) x 2 (tokens), each wave 64 weight
// rows x 80 tokens = 4 x 5 MFMA blocks.  The two-term activations cost 2
// bytes per element (hi + lo) against the weights' half byte, so the tile is
// wide along the weights: per 128-K chunk a workgroup stages 75 KB of
// operands for 2 x 160 x 512 x 128 MACs.  Four waves per SIMD hide each
// other's LDS reads behind their MFMAs, and sixteen waves keep enough
// direct-to-LDS loads in flight (eight waves cap them near 3.7 TB/s on
// gfx950).  Row tiles of up to 160 rows give an expert of 129-320 rows two
// tiles instead of three, the last of a few rows that would cost a full
// tile's weight stream.
constexpr int kSplitTileM = 160;
constexpr int kSplitTokBlocks = kSplitTileM / 32;  // 16-row token blocks per token wave
constexpr int kSplitTileW = 512;
constexpr int kSplitThreads = 1024;
constexpr int kSplitWaves = kSplitThreads / 64;
constexpr int kSplitStages = 2;  // double buffer: chunk c + 1 lands while c is consumed

// LDS stage (one 128-K chunk):
//   activations  two-term formats [160 rows][hi 128 B | lo 128 B], piece p of
//                row R at p ^ (R & 15); ACT_FP4 [160 rows][64 B], piece p of
//                row R at p ^ ((R >> 1) & 3)
//   act. scales  [terms][160 rows] u32 (the chunk's 4 E8M0 bytes), padded to
//                a multiple of 64 slots
//   weights      32 blocks of 16 rows x 64 B, each a tile-major block of the
//                bank as loaded: row 16 b + r, group q at 1024 b + 16 (r + 16 q)
//   w. scales    [512 rows] u32
template <int AF>
struct SplitStage {
  static constexpr int kParts = act_terms(AF);
  static constexpr int kXRow = AF == ACT_FP4 ? 64 : 256;
  static constexpr int kXPieces = kXRow / 16;
  static constexpr int kTermChunk = AF == ACT_FP4 ? 64 : 128;  // stored bytes per row and chunk
  static constexpr int kXBytes = kSplitTileM * kXRow;
  static constexpr int kXSRows = kParts * kSplitTileM;          // real scale slots
  static constexpr int kXSLanes = (kXSRows + 63) / 64 * 64;      // 320 or 192
  static constexpr int kXSBytes = kXSLanes * 4;
  static constexpr int kWBytes = kSplitTileW * 64;
  static constexpr int kWSBytes = kSplitTileW * 4;
  static constexpr int kX = 0, kXS = kXBytes, kW = kXS + kXSBytes, kWS = kW + kWBytes;
  static constexpr int kBytes = kWS + kWSBytes;
  // 1 KB wave loads of the activations (40 or 10): load j of wave w is wave
  // load 16 j + w, issued when it exists
  static constexpr int kXSlots = kXBytes / 1024;
  static constexpr int kXLoads = (kXSlots + kSplitWaves - 1) / kSplitWaves;  // 3 or 1
  static constexpr int kWLoads = kWBytes / (kSplitThreads * 16);             // 2
  // the MFMA's B format of the hi and the lo term (0 E4M3, 2 E2M3, 4 E2M1)
  static constexpr int kMfmaFmt = AF == ACT_FP8X2 || AF == ACT_FP8FP6 ? 0 : (AF == ACT_FP6X2 ? 2 : 4);
  static constexpr int kMfmaFmtLo = AF == ACT_FP8FP6 ? 2 : kMfmaFmt;
  static_assert(kSplitStages * kBytes <= 160 * 1024, "LDS stages exceed 160 KB");
  static_assert(kXBytes % 1024 == 0, "activation loads");
  static_assert(kWSBytes == 8 * 256 && kXSLanes <= 8 * 64, "scale loads per wave");
  static_assert(kSplitWaves * 16 * 144 <= kBytes, "the down epilogue's staging fits a stage");
  __device__ static int xswz(int row) { return kXPieces == 16 ? (row & 15) : ((row >> 1) & 3); }
};

typedef int glm_i32x8 __attribute__((ext_vector_type(8)));

template <int NPROJ, int AF>
__global__ __launch_bounds__(kSplitThreads) void grouped_f8f6f4_kernel(SplitArgs a) {
  using S = SplitStage<AF>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nft = a.feature_tiles;
  // a count above the list's length is clamped to it, so no entry past
  // `tiles` is read and every item still has a workgroup in the grid
  const int ntiles = max(0, min(*a.num_tiles, a.max_tiles));
  const int items = ntiles * nft;
  const int lin = blockIdx.x;
  const int per_xcd = (items + kXcds - 1) / kXcds;
  const int k_on_xcd = lin / kXcds;
  const int item = (lin % kXcds) * per_xcd + k_on_xcd;
  if (k_on_xcd >= per_xcd || item >= items) return;
  const int tile_id = item / nft, ftile = item % nft;
  const int4 tile = a.tiles[tile_id];
  // an empty tile, or one with a negative expert or position, has no work
  // (glm_moe_tiles writes none; the check keeps a caller's list in bounds)
  if (tile.z <= 0 || tile.x < 0 || tile.y < 0) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform copy
  const int wf = wv & 7, wt = wv >> 3;
  const long long e = tile.x;
  // (a tile list from glm_moe_tiles has at most kSplitTileM rows a tile; a
  // longer tile from elsewhere is cut there, so no row past the staged ones
  // is read or stored)
  const int pos0 = tile.y, rows = min(tile.z, kSplitTileM);
  const int K = a.K;
  const int nchunks = K / 128;
  constexpr int kHalf = kSplitTileW / 2;
  const int f0 = ftile * (kSplitTileW / NPROJ);
  auto act_row = [&](int row) -> uint32_t {
    const int pos = pos0 + (row < rows ? row : 0);  // past the end: re-read row 0
    return (uint32_t)(a.act_index != nullptr ? a.act_index[pos] : pos);
  };
  auto w_feature = [&](int row) { return f0 + (NPROJ == 2 ? row % kHalf : row); };

  // ---- load assignment (fixed over the K loop).  Load j of wave w fills the
  // (j * 16 + w)-th 1 KB block of its region.  Bases are wave-uniform buffer
  // resources, per-lane offsets 32-bit; the chunk advances the uniform offset.
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.xhi, a.split_bytes);
  const uint32_t lo_off = (uint32_t)(a.xlo - a.xhi);
  const uint32_t code_row = (uint32_t)act_code_row(K, AF);
  uint32_t xoff[S::kXLoads];
#pragma unroll
  for (int j = 0; j < S::kXLoads; ++j) {
    const int slot = (j * kSplitWaves + wave) * 64 + lane;
    const int row = (slot / S::kXPieces) % kSplitTileM;  // (loads past kXSlots: never issued)
    const int piece = (slot % S::kXPieces) ^ S::xswz(row);
    xoff[j] = act_row(row) * code_row +
              (S::kParts == 2 ? (piece < 8 ? 0u : lo_off) + (piece & 7) * 16 : piece * 16);
  }
  // weight load j of wave w stages rows 16 g .. 16 g + 15, g = 16 j + w (load
  // j: one projection's 256 rows): the bank's tile-major block of those 16
  // features and the chunk, 1 KB of contiguous memory (chunk c at c KB)
  const uint32_t wproj_bytes = (uint32_t)a.N * (uint32_t)(K / 2);
  __amdgpu_buffer_rsrc_t wrs[S::kWLoads];
  uint32_t woff[S::kWLoads];
#pragma unroll
  for (int j = 0; j < S::kWLoads; ++j) {
    const int g = j * kSplitWaves + wave;
    wrs[j] = make_rsrc(a.w[NPROJ == 2 ? j : 0] + e * a.w_stride, wproj_bytes);
    woff[j] = (uint32_t)(w_feature(16 * g) / 16) * (uint32_t)(K / 128) * 1024u + 16u * lane;
  }
  static_assert(S::kWLoads == 2 && kSplitWaves * 64 / 4 == kHalf, "one projection per load");
  // one scale dword per thread: waves 0-7 the weight scales (64 rows each);
  // waves 8-15 the activation scales, slot s = term * 160 + row, repeated
  // once the slots run out (every wave issues the same count); the padding
  // slots past the real ones load slot 0's scale
  __amdgpu_buffer_rsrc_t srs;
  uint32_t soff;
  int sdst;
  if (wv < 8) {
    // weight scales: waves 0-3 the first 256 staged rows, 4-7 the second
    const int row = wv * 64 + lane;
    srs = make_rsrc(a.s[NPROJ == 2 && wv >= 4 ? 1 : 0] + e * a.s_stride,
                    (uint32_t)a.N * (uint32_t)(K / 32));
    soff = (uint32_t)w_feature(row) * (uint32_t)(K / 32);
    sdst = S::kWS + wv * 256;
  } else {
    const int s0 = ((wv - 8) * 64) % S::kXSLanes;
    const int s = s0 + lane < S::kXSRows ? s0 + lane : 0;
    srs = xrs;
    soff = (uint32_t)((s >= kSplitTileM ? a.xslo : a.xshi) - a.xhi) +
           act_row(s % kSplitTileM) * (uint32_t)(K / 32);
    sdst = S::kXS + s0 * 4;
  }

  auto issue = [&](int c, int stage) {
    uint8_t *base = smem + stage * S::kBytes;
#pragma unroll
    for (int j = 0; j < S::kXLoads; ++j)
      if (j * kSplitWaves + wv < S::kXSlots)
        buf16_to_lds(xrs, base + S::kX + (j * kSplitWaves + wv) * 1024, xoff[j],
                     c * S::kTermChunk);
#pragma unroll
    for (int j = 0; j < S::kWLoads; ++j)
      buf16_to_lds(wrs[j], base + S::kW + (j * kSplitWaves + wv) * 1024, woff[j], c * 1024);
    buf4_to_lds(srs, base + sdst, soff, c * 4);
  };

  // this wave's weight-row blocks: 4 of 16 rows (gate/up: 2 gate blocks, then
  // the 2 up blocks of the same features)
  auto wrow_of = [&](int rt) {
    return NPROJ == 2 ? (rt / 2) * kHalf + wf * 32 + (rt % 2) * 16 : wf * 64 + rt * 16;
  };

  // the tile's 16-row token blocks are split evenly between the two token
  // waves (wave 0 takes the odd one), so the four waves of a SIMD issue
  // about as many MFMAs each; blocks past the tile's rows are skipped (their
  // columns are never stored)
  constexpr int kTB = kSplitTokBlocks;
  const int half = 16 * ((((rows + 15) >> 4) + 1) >> 1);
  const int tok0 = wt ? half : 0;     // the wave's first token row
  const int tend = wt ? rows : half;  // and the end of its blocks (<= tok0 + 16 kTB)
  glm_f32x4 acc[4][kTB];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kTB; ++j) acc[i][j] = glm_f32x4{0.f, 0.f, 0.f, 0.f};

  // Lane-dependent parts of the LDS operand addresses.  Every block starts at
  // a multiple of 16 rows, so a lane's swizzle depends on r alone: two-term
  // activation row 16m + r, piece p at (16m + r) * 256 + 16 (p ^ r); ACT_FP4
  // row 16m + r, piece p at (16m + r) * 64 + 16 (p ^ ((r >> 1) & 3)); weight
  // row 16m + r, group q at 1024 m + 16 (r + 16 q).
  uint32_t xl[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    xl[t][0] = r * S::kXRow + 16 * (S::kParts == 2 ? ((8 * t + q) ^ r) : (q ^ ((r >> 1) & 3)));
    xl[t][1] = r * S::kXRow + 16 * ((8 * t + 4 + q) ^ r);
  }
  const uint32_t wl = 16 * r + 256 * q;
  const uint32_t sl = r * 4;

  // MFMAs of one staged chunk: for each activation fragment (term x 5 token
  // blocks) 4 MFMAs, one per weight-row block.
  auto compute = [&](int stage) {
    const uint8_t *base = smem + stage * S::kBytes;
    glm_i32x8 wa[4];
    int wsc[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int w16 = wrow_of(rt);  // first row of the block
      const glm_u32x4 v = *reinterpret_cast<const glm_u32x4 *>(base + S::kW + w16 * 64 + wl);
      wa[rt] = glm_i32x8{(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
      wsc[rt] = (int)(*reinterpret_cast<const uint32_t *>(base + S::kWS + w16 * 4 + sl) >> (8 * q));
    }
    // activation fragment f = (term f / kTB, token block f % kTB)
    constexpr int kFrags = kTB * S::kParts;
    auto xfrag = [&](int f, glm_i32x8 &xb, int &xsc) {
      const int t = f / kTB, ct = f % kTB;
      const uint8_t *xblk = base + S::kX + (tok0 + ct * 16) * S::kXRow;
      const glm_u32x4 b0 = *reinterpret_cast<const glm_u32x4 *>(xblk + xl[t][0]);
      if constexpr (S::kParts == 2) {
        const glm_u32x4 b1 = *reinterpret_cast<const glm_u32x4 *>(xblk + xl[t][1]);
        xb = glm_i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3],
                       (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
      } else {
        xb = glm_i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], 0, 0, 0, 0};
      }
      xsc = (int)(*reinterpret_cast<const uint32_t *>(
                      base + S::kXS + (t * kSplitTileM + tok0 + ct * 16) * 4 + sl) >>
                  (8 * q));
    };
#pragma unroll
    for (int f = 0; f < kFrags; ++f) {
      if (tok0 + (f % kTB) * 16 < tend) {
        glm_i32x8 xb;
        int xsc;
        xfrag(f, xb, xsc);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          if (f < kTB)
            acc[rt][f % kTB] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                wa[rt], xb, acc[rt][f % kTB], 4, S::kMfmaFmt, 0, wsc[rt], 0, xsc);
          else
            acc[rt][f % kTB] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                wa[rt], xb, acc[rt][f % kTB], 4, S::kMfmaFmtLo, 0, wsc[rt], 0, xsc);
        }
      }
    }
  };

  // Double buffer: the loads of chunk c + 1 are issued after the barrier that
  // follows every wave's chunk c - 1 (whose stage they overwrite) and land
  // while chunk c is consumed.
  issue(0, 0);
  for (int c = 0; c < nchunks; ++c) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    ring_barrier();
    if (c + 1 < nchunks) issue(c + 1, (c + 1) % kSplitStages);
    compute(c % kSplitStages);
  }

  // SwiGLU of the gate/up sums m, m + 1 of one accumulator pair (gate block,
  // up block), each projection rounded to bf16 first
  const float lim = a.limit > 0.0f ? a.limit : __builtin_inff();
  auto swiglu_pair = [&](const glm_f32x4 &g, const glm_f32x4 &u, int m, float &h0, float &h1) {
    float g0 = g[m], g1 = g[m + 1], u0 = u[m], u1 = u[m + 1];
    bf16_round2(g0, g1);
    bf16_round2(u0, u1);
    limited_swiglu2_fast(g0, g1, u0, u1, lim, h0, h1);
  };

  // ---- epilogue: lane (r, q) of block (rt, ct) holds weight rows 4q..4q+3 of
  // the block for token column r
  if constexpr (NPROJ == 2 && AF == ACT_FP8X2) {
    if (a.out_split != nullptr) {
      // h's FP8 hi/lo split, exactly as act_split_kernel forms it from the
      // bf16 h: the wave's 32 features f0 + 32 wf + [0, 32) of a token are one
      // scale group, held 8 per lane by the four lanes (r, q = 0..3); the
      // group maxima are exchanged across them (the shuffles run on every
      // lane, the stores only for real rows)
      const SplitLayout L(a.out_rows, a.N);
      const int g0 = f0 + wf * 32;
#pragma unroll
      for (int ct = 0; ct < kTB; ++ct) {
        if (tok0 + ct * 16 >= tend) continue;
        const int row = tok0 + ct * 16 + r;
        float v[8];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int m = 0; m < 4; m += 2)
            swiglu_pair(acc[i][ct], acc[2 + i][ct], m, v[4 * i + m], v[4 * i + m + 1]);
        uint32_t ch[2], cl[2];
        int bh, bl;
        split_group_part(v, ch, cl, &bh, &bl);
        if (row < rows) {
          const size_t prow = (size_t)(pos0 + row);
          uint8_t *hi = a.out_split + prow * a.N + g0;
          uint8_t *lo = a.out_split + L.lo + prow * a.N + g0;
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            *reinterpret_cast<uint32_t *>(hi + i * 16 + 4 * q) = ch[i];
            *reinterpret_cast<uint32_t *>(lo + i * 16 + 4 * q) = cl[i];
          }
          if (q == 0) {
            a.out_split[L.shi + prow * (a.N / 32) + g0 / 32] = (uint8_t)bh;
            a.out_split[L.slo + prow * (a.N / 32) + g0 / 32] = (uint8_t)bl;
          }
        }
      }
      return;
    }
  }
  if constexpr (NPROJ == 2) {
#pragma unroll
    for (int ct = 0; ct < kTB; ++ct) {
      const int row = tok0 + ct * 16 + r;
      if (tok0 + ct * 16 >= tend || row >= rows) continue;
      uint16_t *orow = a.out + (size_t)(pos0 + row) * a.N;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        float h[4];
        swiglu_pair(acc[i][ct], acc[2 + i][ct], 0, h[0], h[1]);
        swiglu_pair(acc[i][ct], acc[2 + i][ct], 2, h[2], h[3]);
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = __float_as_uint(h[m]) >> 16;  // bf16-exact
        store_rows4(orow + f0 + wf * 32 + i * 16 + 4 * q, o);
      }
    }
  } else {
    // y through LDS, so that every store writes whole 128-byte lines: per
    // token block the wave's 16 rows x 64 features go to its own 16 x 144 B
    // area of the stage no chunk occupies (the ring's last loads went to the
    // other one), and come back as 16 contiguous bytes per lane, 8 lanes a
    // row.  (Stored straight from the accumulators each instruction wrote
    // 8 bytes into each of 16 rows.)
    uint8_t *yst = smem + (nchunks % kSplitStages) * S::kBytes + wv * (16 * 144);
    const int rr = lane >> 3, seg = lane & 7;
#pragma unroll
    for (int ct = 0; ct < kTB; ++ct) {
      if (tok0 + ct * 16 >= tend) continue;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = f32_to_bf16(acc[rt][ct][m]);
        *reinterpret_cast<uint2 *>(yst + r * 144 + (rt * 16 + 4 * q) * 2) =
            uint2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = tok0 + ct * 16 + 8 * h + rr;
        const glm_u32x4 v = *reinterpret_cast<const glm_u32x4 *>(yst + (8 * h + rr) * 144 + 16 * seg);
        if (row < rows)
          *reinterpret_cast<glm_u32x4 *>(a.out + (size_t)(pos0 + row) * a.N + f0 + wf * 64 + 8 * seg) = v;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

// ---------------------------------------------------------------------------
// Eight-wave form of the block-scaled GEMMs: the same workgroup tile (up to
// 160 dispatch rows x 512 weight rows), LDS stage and direct-to-LDS loads as
// grouped_f8f6f4_kernel, computed by 8 waves of up to 256 registers (two per
// SIMD) as 4 (weight rows) x 2 (tokens): each wave owns 128 weight rows x up
// to 80 tokens = 8 x 5 MFMA blocks.  Every activation fragment read from LDS
// then feeds 8 MFMAs instead of 4 (229 KB of operand reads per chunk and
// workgroup instead of 393 KB), and the registers leave room to read
// fragment f + 1 while the MFMAs of fragment f run; with the exact FP8 split
// the next chunk's weights and first fragment are read behind the last
// MFMAs of the chunk before, after the barrier that releases them.  The body is
// instantiated per count NB of the wave's 16-row token blocks (0..5), so every
// fragment and accumulator index is static.
// ---------------------------------------------------------------------------
constexpr int kW8Threads = 512;
constexpr int kW8Waves = kW8Threads / 64;
constexpr int kW8YRow = 272;  // bytes per row of the down epilogue's staging (256 + 16)

// LDS of the eight-wave form: the two stages' parts side by side (all
// activation codes, then all weight codes, weight scales, activation scales),
// so that every operand read is a per-lane base register plus an immediate
// offset below 64 KB.
template <int AF>
struct W8Layout {
  using S = SplitStage<AF>;
  static constexpr int kX = 0;
  static constexpr int kW = kX + kSplitStages * S::kXBytes;
  static constexpr int kWS = kW + kSplitStages * S::kWBytes;
  static constexpr int kXS = kWS + kSplitStages * S::kWSBytes;
  // the row table: one u32 per row any activation load can name (rows past
  // the tile's hold row 0's offset)
  static constexpr int kTabRows =
      (S::kXSlots + kW8Waves - 1) / kW8Waves * kW8Waves * (64 / S::kXPieces);
  static constexpr int kRows = kXS + kSplitStages * S::kXSBytes;  // u32 [kTabRows]
  static constexpr int kBytes = kRows + kTabRows * 4;
  static_assert(kRows == kSplitStages * S::kBytes, "the stages as in the stage layout");
  static_assert(kBytes <= 160 * 1024, "LDS exceeds 160 KB");
  static_assert((kSplitStages - 1) * S::kXBytes + (kSplitTileM / 2) * S::kXRow < 65536 &&
                    (kSplitStages - 1) * S::kWBytes + S::kWBytes - 1024 < 65536,
                "operand offsets fit the 16-bit LDS immediate");
  static_assert(kW8Waves * 16 * kW8YRow <= kBytes, "the down epilogue's staging fits");
};

template <int N>
struct W8Stage {
  static constexpr int value = N;
};

// N dwords from LDS at base + j * STEP (j < N, 2 or 5) into v, then a wait
// for every LDS access of the wave in flight (lgkmcnt(0)), in one asm
// statement: the compiler sees v defined only once the reads have landed, so
// it never copies or spills a register that the LDS has yet to write.
template <int N, int STEP>
__device__ __forceinline__ void lds_rows(uint32_t *v, uint32_t base) {
  static_assert((N == 2 || N == 5) && (N - 1) * STEP < 65536, "row table reads");
  if constexpr (N == 2)
    asm volatile(
        "ds_read_b32 %0, %2\n\t"
        "ds_read_b32 %1, %2 offset:%3\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1])
        : "v"(base), "i"(STEP)
        : "memory");
  else
    asm volatile(
        "ds_read_b32 %0, %5\n\t"
        "ds_read_b32 %1, %5 offset:%6\n\t"
        "ds_read_b32 %2, %5 offset:%7\n\t"
        "ds_read_b32 %3, %5 offset:%8\n\t"
        "ds_read_b32 %4, %5 offset:%9\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4])
        : "v"(base), "i"(STEP), "i"(2 * STEP), "i"(3 * STEP), "i"(4 * STEP)
        : "memory");
}

template <int NPROJ, int AF, int NB>
__device__ __forceinline__ void w8_body(const SplitArgs &a, long long e, int pos0, int rows,
                                        int ftile, int tok0) {
  using S = SplitStage<AF>;
  using L = W8Layout<AF>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int r = lane & 15, q = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wf = wv & 3;
  const int K = a.K;
  const int nchunks = K / 128;
  constexpr int kHalf = kSplitTileW / 2;
  const int f0 = ftile * (kSplitTileW / NPROJ);
  auto act_row = [&](int row) -> uint32_t {
    const int pos = pos0 + (row < rows ? row : 0);  // past the end: re-read row 0
    return (uint32_t)(a.act_index != nullptr ? a.act_index[pos] : pos);
  };

  // ---- load assignment (fixed over the K loop), as grouped_f8f6f4_kernel's
  // with 8 waves: activation wave load j * 8 + w; weight block g = j * 8 + w
  // (loads 0-1 the first projection's 256 rows, 2-3 the second's); weight
  // scale rows 64 w .. 64 w + 63; activation scale slots 64 w .. 64 w + 63.
  // Only the activation rows are per lane; the weight offsets are a lane
  // term plus a uniform one.
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.xhi, a.split_bytes);
  const uint32_t lo_off = (uint32_t)(a.xlo - a.xhi);
  const uint32_t code_row = (uint32_t)act_code_row(K, AF);
  // Activation wave load j of wave w covers rows R_j = (8 j + w) 64 / kXPieces
  // + lane / kXPieces; the lane's piece is the same for every j (the row's
  // swizzle bits do not depend on j), so a load's offset is the code-row
  // offset of R_j, from a table of the tile's rows in LDS, plus one per-lane
  // piece offset.
  constexpr int kXL = (S::kXSlots + kW8Waves - 1) / kW8Waves;  // 5 or 2
  constexpr int kRowsPerLoad = 64 / S::kXPieces;
  uint32_t xpiece;
  {
    const int row = (wv * 64 + lane) / S::kXPieces;
    const int piece = (lane % S::kXPieces) ^ S::xswz(row);
    xpiece = S::kParts == 2 ? (piece < 8 ? 0u : lo_off) + (piece & 7) * 16 : piece * 16;
  }
  const uint32_t xtab = (uint32_t)(L::kRows + 4 * (wv * kRowsPerLoad + lane / S::kXPieces));
  static_assert(L::kTabRows == kXL * kW8Waves * kRowsPerLoad && L::kTabRows >= kSplitTileM,
                "the row table covers every load");
  for (int i = threadIdx.x; i < L::kTabRows; i += kW8Threads)
    reinterpret_cast<uint32_t *>(smem + L::kRows)[i] = act_row(i) * code_row;
  constexpr int kWL = S::kWBytes / (kW8Threads * 16);
  static_assert(kWL == 4, "two weight loads per projection");
  const uint32_t wproj_bytes = (uint32_t)a.N * (uint32_t)(K / 2);
  const __amdgpu_buffer_rsrc_t wrs0 = make_rsrc(a.w[0] + e * a.w_stride, wproj_bytes);
  const __amdgpu_buffer_rsrc_t wrs1 = make_rsrc(a.w[NPROJ == 2 ? 1 : 0] + e * a.w_stride,
                                                wproj_bytes);
  const uint32_t wlane = 16u * lane;
  uint32_t wuni[kWL];  // the block's first feature / 16 x the bytes of a block row
#pragma unroll
  for (int j = 0; j < kWL; ++j) {
    const int g = j * kW8Waves + wv;
    const int feat = f0 + (NPROJ == 2 ? (16 * g) % kHalf : 16 * g);
    wuni[j] = (uint32_t)(feat / 16) * (uint32_t)(K / 128) * 1024u;
  }
  const __amdgpu_buffer_rsrc_t wsrs =
      make_rsrc(a.s[NPROJ == 2 && wv >= 4 ? 1 : 0] + e * a.s_stride,
                (uint32_t)a.N * (uint32_t)(K / 32));
  const uint32_t wslane = (uint32_t)lane * (uint32_t)(K / 32);
  const uint32_t wsuni =
      (uint32_t)(f0 + (NPROJ == 2 ? (wv * 64) % kHalf : wv * 64)) * (uint32_t)(K / 32);
  // every wave loads 64 scale slots (wave w: slots 64 w mod the padded
  // count, so waves past the last slot repeat earlier ones with the same
  // bytes); padding slots load slot 0's scale
  const int xs0 = (wv * 64) % S::kXSLanes;
  uint32_t xsoff;
  {
    const int s = xs0 + lane < S::kXSRows ? xs0 + lane : 0;
    xsoff = (uint32_t)((s >= kSplitTileM ? a.xslo : a.xshi) - a.xhi) +
            act_row(s % kSplitTileM) * (uint32_t)(K / 32);
  }

  // The loads of chunk c into stage ST.  The activation rows' offsets come
  // from the row table in LDS, read as explicit instructions (one base
  // register, immediate offsets; a compiler-generated read keeps one address
  // register per load live across the loop).
  auto table_rows = [&](uint32_t *xrow) { lds_rows<kXL, 4 * kW8Waves * kRowsPerLoad>(xrow, xtab); };
  auto issue_loads = [&](auto st, int c, const uint32_t *xrow) {
    constexpr int ST = decltype(st)::value;
#pragma unroll
    for (int j = 0; j < kWL; ++j)
      buf16_to_lds(j < 2 ? wrs0 : wrs1, smem + L::kW + ST * S::kWBytes + (j * kW8Waves + wv) * 1024,
                   wlane, wuni[j] + c * 1024);
#pragma unroll
    for (int j = 0; j < kXL; ++j)
      if (S::kXSlots % kW8Waves == 0 || j * kW8Waves + wv < S::kXSlots)
        buf16_to_lds(xrs, smem + L::kX + ST * S::kXBytes + (j * kW8Waves + wv) * 1024,
                     xrow[j] + xpiece, c * S::kTermChunk);
    buf4_to_lds(wsrs, smem + L::kWS + ST * S::kWSBytes + wv * 256, wslane, wsuni + c * 4);
    buf4_to_lds(xrs, smem + L::kXS + ST * S::kXSBytes + xs0 * 4, xsoff, c * 4);
  };


  glm_f32x4 acc[8][NB > 0 ? NB : 1];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < (NB > 0 ? NB : 1); ++j) acc[i][j] = glm_f32x4{0.f, 0.f, 0.f, 0.f};

  // Per-lane LDS bases.  Activation row tok0 + 16 ct + r, piece p at
  // row * kXRow + 16 (p ^ swizzle(r)): the term-t, half-h piece of the
  // two-term formats, p = 8 t + 4 h + q, lies at xl ^ 64 (2 t + h) (the row
  // part is a multiple of 256); ACT_FP4's piece q at xl.  Weight block b,
  // group q of row r at 1024 b + 16 lane; scale bytes at 4 row + q.
  static_assert((L::kX % 256 == 0 && S::kXRow % 256 == 0) || S::kParts == 1, "xor addressing");
  const uint32_t xl = (uint32_t)(L::kX + (tok0 + r) * S::kXRow +
                                 16 * (S::kParts == 2 ? (q ^ r) : (q ^ ((r >> 1) & 3))));
  const uint32_t wl = (uint32_t)L::kW + wlane;
  const uint32_t wsl = (uint32_t)(L::kWS + 4 * r + q);
  const uint32_t xsl = (uint32_t)(L::kXS + 4 * (tok0 + r) + q);

  // Operand registers carried from one chunk to the next: the chunk's eight
  // weight blocks (their scale bytes packed four to a register; the MFMA's
  // byte select picks one) and two activation fragments, the one whose MFMAs
  // run and the next.  Fragment f of a chunk is term f / NB, token block
  // f % NB, held in xb[(f + P) & 1] for the chunk's parity P.
  constexpr int kFrags = NB * S::kParts;
  glm_i32x8 xb[2];
  int xsc[2];
  glm_i32x8 wa[8];
  int wsp[2];
  auto xfrag = [&](auto st, int f, glm_i32x8 &xbv, int &xs) {
    constexpr int ST = decltype(st)::value;
    const int t = f / NB, ct = f % NB;
    constexpr int kXo = ST * S::kXBytes;
    const int co = kXo + ct * 16 * S::kXRow;
    const glm_u32x4 b0 = *reinterpret_cast<const glm_u32x4 *>(smem + (xl ^ (128u * t)) + co);
    if constexpr (S::kParts == 2) {
      const glm_u32x4 b1 = *reinterpret_cast<const glm_u32x4 *>(smem + (xl ^ (128u * t + 64u)) + co);
      xbv = glm_i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3],
                      (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    } else {
      xbv = glm_i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], 0, 0, 0, 0};
    }
    xs = smem[xsl + ST * S::kXSBytes + 4 * (t * kSplitTileM + ct * 16)];
  };
  // Weight block i of the wave (codes into w) and its scale byte.  The
  // wave's eight blocks (16 rows each) index the stage's 32 as
  // kWfBlocks * wf + boff(i): gate/up 4 gate blocks (features 64 wf ..
  // 64 wf + 63), then the 4 up blocks of the same features; down 8
  // consecutive blocks.  Each is read at one per-lane base plus an immediate
  // offset.
  constexpr int kWfBlocks = NPROJ == 2 ? 4 : 8;
  auto boff = [](int i) { return NPROJ == 2 && i >= 4 ? i + 12 : i; };
  const uint8_t *wbase = smem + wl + (uint32_t)(kWfBlocks * 1024) * (uint32_t)wf;
  const uint8_t *wsbase = smem + wsl + (uint32_t)(kWfBlocks * 64) * (uint32_t)wf;
  auto wread = [&](auto st, int i, glm_i32x8 &w) -> uint32_t {
    constexpr int ST = decltype(st)::value;
    const glm_u32x4 v =
        *reinterpret_cast<const glm_u32x4 *>(wbase + ST * S::kWBytes + boff(i) * 1024);
    w = glm_i32x8{(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
    return wsbase[ST * S::kWSBytes + boff(i) * 64];
  };
  // the MFMA of fragment f with weight block B (the byte select must be a
  // constant, hence one instantiation per block)
  auto mf = [&](auto bt, int f, const glm_i32x8 &xv, int xs) {
    constexpr int B = decltype(bt)::value;
    const int ct = f % NB;
    if (f < NB)
      acc[B][ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
          wa[B], xv, acc[B][ct], 4, S::kMfmaFmt, B & 3, wsp[B >> 2], 0, xs);
    else
      acc[B][ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
          wa[B], xv, acc[B][ct], 4, S::kMfmaFmtLo, B & 3, wsp[B >> 2], 0, xs);
  };
  auto mf8 = [&](int f, const glm_i32x8 &xv, int xs) {
    mf(W8Stage<0>{}, f, xv, xs);
    mf(W8Stage<1>{}, f, xv, xs);
    mf(W8Stage<2>{}, f, xv, xs);
    mf(W8Stage<3>{}, f, xv, xs);
    mf(W8Stage<4>{}, f, xv, xs);
    mf(W8Stage<5>{}, f, xv, xs);
    mf(W8Stage<6>{}, f, xv, xs);
    mf(W8Stage<7>{}, f, xv, xs);
  };
  // a chunk's weight blocks, scales and first fragment (parity P)
  auto read_head = [&](auto st, auto par) {
    constexpr int P = decltype(par)::value;
    xfrag(st, 0, xb[P], xsc[P]);
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      uint32_t sb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sb[i] = wread(st, 4 * hb + i, wa[4 * hb + i]);
      wsp[hb] = (int)(sb[0] | (sb[1] << 8) | (sb[2] << 16) | (sb[3] << 24));
    }
  };

  // The MFMAs of the chunk in stage ST (parity P), its head already in
  // registers: each fragment's 8 MFMAs run while the next fragment is read.
  // Before the last fragment's MFMAs the wave waits for its own loads of the
  // next chunk and for its reads of this stage, and meets the other waves at
  // the barrier: after it every wave's loads of the next chunk have landed
  // and no wave reads this stage again.  The next chunk's head is then read
  // into the registers that the last fragment's MFMAs free, one weight block
  // behind each MFMA, so the next chunk's first MFMAs need not wait for a
  // burst of reads after the barrier.
  auto run_chunk = [&](auto st, auto par, auto nx) {
    constexpr int ST = decltype(st)::value, P = decltype(par)::value;
    constexpr int kNx = decltype(nx)::value;  // 1: a next chunk follows
    constexpr int L = kFrags - 1;
    // fragments 0 .. L - 2, each with the next one read ahead; the read of
    // fragment L is the chunk's last access to its stage
#pragma unroll
    for (int f = 0; f + 1 < L; ++f) {
      xfrag(st, f + 1, xb[(f + 1 + P) & 1], xsc[(f + 1 + P) & 1]);
      mf8(f, xb[(f + P) & 1], xsc[(f + P) & 1]);
    }
    if constexpr (L >= 1) xfrag(st, L, xb[(L + P) & 1], xsc[(L + P) & 1]);
#pragma unroll
    for (int f = 0; f + 1 < L; ++f) {
      __builtin_amdgcn_sched_group_barrier(0x100, S::kParts + 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    }
    if constexpr (L >= 1) __builtin_amdgcn_sched_group_barrier(0x100, S::kParts + 1, 0);
    if constexpr (kNx > 0) {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & ~(15 << 8));  // vmcnt(0) lgkmcnt(0)
      ring_barrier();
      if constexpr (L >= 1) mf8(L - 1, xb[(L - 1 + P) & 1], xsc[(L - 1 + P) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      constexpr W8Stage<1 - ST> ns{};
      constexpr int NP = (P + kFrags) & 1;
      const glm_i32x8 xv = xb[(L + P) & 1];
      const int xs = xsc[(L + P) & 1];
      uint32_t sb[8];
      mf(W8Stage<0>{}, L, xv, xs);
      sb[0] = wread(ns, 0, wa[0]);
      mf(W8Stage<1>{}, L, xv, xs);
      sb[1] = wread(ns, 1, wa[1]);
      mf(W8Stage<2>{}, L, xv, xs);
      sb[2] = wread(ns, 2, wa[2]);
      mf(W8Stage<3>{}, L, xv, xs);
      sb[3] = wread(ns, 3, wa[3]);
      mf(W8Stage<4>{}, L, xv, xs);
      sb[4] = wread(ns, 4, wa[4]);
      mf(W8Stage<5>{}, L, xv, xs);
      sb[5] = wread(ns, 5, wa[5]);
      mf(W8Stage<6>{}, L, xv, xs);
      sb[6] = wread(ns, 6, wa[6]);
      mf(W8Stage<7>{}, L, xv, xs);
      sb[7] = wread(ns, 7, wa[7]);
      xfrag(ns, 0, xb[NP], xsc[NP]);
      wsp[0] = (int)(sb[0] | (sb[1] << 8) | (sb[2] << 16) | (sb[3] << 24));
      wsp[1] = (int)(sb[4] | (sb[5] << 8) | (sb[6] << 16) | (sb[7] << 24));
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, S::kParts + 1, 0);
    } else {
      if constexpr (L >= 1) mf8(L - 1, xb[(L - 1 + P) & 1], xsc[(L - 1 + P) & 1]);
      mf8(L, xb[(L + P) & 1], xsc[(L + P) & 1]);
    }
  };

  // Double buffer, unrolled by two so that each stage's offsets are
  // immediates: the loads of chunk c + 1 are issued at the top of chunk c,
  // into the stage of chunk c - 1 (free since the barrier inside chunk
  // c - 1), and land while chunk c is consumed.  A wave without token blocks
  // issues its loads and meets the same barriers.
  ring_barrier();  // the row table
  {
    uint32_t xrow[kXL];
    table_rows(xrow);
    issue_loads(W8Stage<0>{}, 0, xrow);
  }
  if constexpr (AF == ACT_FP8X2) {
    // The exact FP8 split: the operands cross the barrier in registers (see
    // run_chunk).  The chunk count is even (K a multiple of 256); the last
    // chunk, which has no next one, is peeled.
    constexpr int kP1 = kFrags & 1;  // parity of the chunks in stage 1
    auto step = [&](auto st, int c, auto nx) {
      constexpr int kNx = decltype(nx)::value;
      constexpr int ST = decltype(st)::value;
      if constexpr (kNx > 0) {
        uint32_t xrow[kXL];
        table_rows(xrow);
        issue_loads(W8Stage<1 - ST>{}, c + 1, xrow);
      }
      if constexpr (NB > 0) {
        run_chunk(st, W8Stage<ST == 0 ? 0 : kP1>{}, nx);
      } else if constexpr (kNx > 0) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & ~(15 << 8));
        ring_barrier();
      }
    };
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    ring_barrier();
    if constexpr (NB > 0) read_head(W8Stage<0>{}, W8Stage<0>{});
    for (int c = 0; c + 2 < nchunks; c += 2) {
      step(W8Stage<0>{}, c, W8Stage<1>{});
      step(W8Stage<1>{}, c + 1, W8Stage<1>{});
    }
    step(W8Stage<0>{}, nchunks - 2, W8Stage<1>{});
    step(W8Stage<1>{}, nchunks - 1, W8Stage<0>{});
  } else {
    // The other formats (their kernels spill with the operands carried in
    // registers): each chunk's head is read after the barrier that releases
    // the chunk, then its fragments with the next one read ahead.
    auto compute = [&](auto st) {
      if constexpr (NB > 0) {
        read_head(st, W8Stage<0>{});
#pragma unroll
        for (int f = 0; f < kFrags; ++f) {
          if (f + 1 < kFrags) xfrag(st, f + 1, xb[(f + 1) & 1], xsc[(f + 1) & 1]);
          mf8(f, xb[f & 1], xsc[f & 1]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, S::kParts + 1 + 16, 0);
#pragma unroll
        for (int f = 0; f < kFrags; ++f) {
          if (f + 1 < kFrags) __builtin_amdgcn_sched_group_barrier(0x100, S::kParts + 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        }
      }
    };
    auto step = [&](auto st, int c) {
      constexpr int ST = decltype(st)::value;
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      ring_barrier();
      if (c + 1 < nchunks) {
        uint32_t xrow[kXL];
        table_rows(xrow);
        issue_loads(W8Stage<1 - ST>{}, c + 1, xrow);
      }
      compute(st);
    };
    for (int c = 0; c < nchunks; c += 2) {
      step(W8Stage<0>{}, c);
      if (c + 1 < nchunks) step(W8Stage<1>{}, c + 1);
    }
  }
  // the down epilogue stages y in LDS that other waves may still read:
  // every wave (also one without token blocks) passes this barrier first
  if constexpr (NPROJ == 1) ring_barrier();
  if constexpr (NB == 0) return;

  const float lim = a.limit > 0.0f ? a.limit : __builtin_inff();
  auto swiglu_pair = [&](const glm_f32x4 &g, const glm_f32x4 &u, int m, float &h0, float &h1) {
    float g0 = g[m], g1 = g[m + 1], u0 = u[m], u1 = u[m + 1];
    bf16_round2(g0, g1);
    bf16_round2(u0, u1);
    limited_swiglu2_fast(g0, g1, u0, u1, lim, h0, h1);
  };

  // ---- epilogue: lane (r, q) of block (b, ct) holds weight rows 4q..4q+3 of
  // the block for token column r
  if constexpr (NPROJ == 2 && AF == ACT_FP8X2) {
    if (a.out_split != nullptr) {
      // h's FP8 hi/lo split (as act_split_kernel forms it from the bf16 h):
      // the wave's 64 features are two scale groups, group gi held 8 per lane
      // by the lanes (r, q = 0..3) in gate/up blocks 2 gi, 2 gi + 1
      const SplitLayout SL(a.out_rows, a.N);
#pragma unroll
      for (int ct = 0; ct < NB; ++ct) {
        const int row = tok0 + ct * 16 + r;
#pragma unroll
        for (int gi = 0; gi < 2; ++gi) {
          float v[8];
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int m = 0; m < 4; m += 2)
              swiglu_pair(acc[2 * gi + i][ct], acc[4 + 2 * gi + i][ct], m, v[4 * i + m],
                          v[4 * i + m + 1]);
          uint32_t ch[2], cl[2];
          int bh, bl;
          split_group_part(v, ch, cl, &bh, &bl);
          if (row < rows) {
            const int g0 = f0 + wf * 64 + gi * 32;
            const size_t prow = (size_t)(pos0 + row);
            uint8_t *hi = a.out_split + prow * a.N + g0;
            uint8_t *lo = a.out_split + SL.lo + prow * a.N + g0;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
              *reinterpret_cast<uint32_t *>(hi + i * 16 + 4 * q) = ch[i];
              *reinterpret_cast<uint32_t *>(lo + i * 16 + 4 * q) = cl[i];
            }
            if (q == 0) {
              a.out_split[SL.shi + prow * (a.N / 32) + g0 / 32] = (uint8_t)bh;
              a.out_split[SL.slo + prow * (a.N / 32) + g0 / 32] = (uint8_t)bl;
            }
          }
        }
      }
      return;
    }
  }
  if constexpr (NPROJ == 2) {
#pragma unroll
    for (int ct = 0; ct < NB; ++ct) {
      const int row = tok0 + ct * 16 + r;
      if (row >= rows) continue;
      uint16_t *orow = a.out + (size_t)(pos0 + row) * a.N;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float h[4];
        swiglu_pair(acc[i][ct], acc[4 + i][ct], 0, h[0], h[1]);
        swiglu_pair(acc[i][ct], acc[4 + i][ct], 2, h[2], h[3]);
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = __float_as_uint(h[m]) >> 16;  // bf16-exact
        store_rows4(orow + f0 + wf * 64 + i * 16 + 4 * q, o);
      }
    }
  } else {
    // y through LDS so that every store writes whole 128-byte lines: per
    // token block the wave's 16 rows x 128 features go to its own 16 x 272 B
    // area and come back as 16 contiguous bytes per lane, 16 lanes a row
    uint8_t *yst = smem + wv * (16 * kW8YRow);
    const int rr = lane >> 4, seg = lane & 15;
#pragma unroll
    for (int ct = 0; ct < NB; ++ct) {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = f32_to_bf16(acc[b][ct][m]);
        *reinterpret_cast<uint2 *>(yst + r * kW8YRow + (b * 16 + 4 * q) * 2) =
            uint2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int row = tok0 + ct * 16 + 4 * h + rr;
        const glm_u32x4 v =
            *reinterpret_cast<const glm_u32x4 *>(yst + (4 * h + rr) * kW8YRow + 16 * seg);
        if (row < rows)
          *reinterpret_cast<glm_u32x4 *>(a.out + (size_t)(pos0 + row) * a.N + f0 + wf * 128 +
                                         8 * seg) = v;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

// One workgroup's work item of the eight-wave form; lin as in bf16_gemm_item.
template <int NPROJ, int AF>
__device__ __forceinline__ void w8_item(const SplitArgs &a, int lin) {
  const int nft = a.feature_tiles;
  // a count above the list's length is clamped to it, so no entry past
  // `tiles` is read and every item still has a workgroup in the grid
  const int ntiles = max(0, min(*a.num_tiles, a.max_tiles));
  const int items = ntiles * nft;
  const int per_xcd = (items + kXcds - 1) / kXcds;
  const int k_on_xcd = lin / kXcds;
  const int item = (lin % kXcds) * per_xcd + k_on_xcd;
  if (k_on_xcd >= per_xcd || item >= items) return;
  const int tile_id = item / nft, ftile = item % nft;
  const int4 tile = a.tiles[tile_id];
  // an empty tile, or one with a negative expert or position, has no work
  // (glm_moe_tiles writes none; the check keeps a caller's list in bounds)
  if (tile.z <= 0 || tile.x < 0 || tile.y < 0) return;
  // (a longer tile than kSplitTileM rows from elsewhere is cut there)
  const int rows = min(tile.z, kSplitTileM);
  // the tile's 16-row token blocks split between the two token waves (wave
  // row 0 takes the odd one); blocks past the tile's rows are not computed
  const int nblk = (rows + 15) >> 4;
  const int half = 16 * ((nblk + 1) >> 1);
  const int wt = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) >> 2;
  const int tok0 = wt ? half : 0;
  const int nb = wt ? nblk - (half >> 4) : (half >> 4);
  switch (nb) {
    case 5: w8_body<NPROJ, AF, 5>(a, tile.x, tile.y, rows, ftile, tok0); break;
    case 4: w8_body<NPROJ, AF, 4>(a, tile.x, tile.y, rows, ftile, tok0); break;
    case 3: w8_body<NPROJ, AF, 3>(a, tile.x, tile.y, rows, ftile, tok0); break;
    case 2: w8_body<NPROJ, AF, 2>(a, tile.x, tile.y, rows, ftile, tok0); break;
    case 1: w8_body<NPROJ, AF, 1>(a, tile.x, tile.y, rows, ftile, tok0); break;
    default: w8_body<NPROJ, AF, 0>(a, tile.x, tile.y, rows, ftile, tok0); break;
  }
}

template <int NPROJ, int AF>
__global__ __launch_bounds__(kW8Threads) void grouped_f8f6f4_w8_kernel(SplitArgs a) {
  w8_item<NPROJ, AF>(a, blockIdx.x);
}

// The routed gate/up (work items of the eight-wave form, workgroups
// [0, routed_blocks)) and the bf16 shared expert's dense gate/up (TW-row
// tiles, the workgroups after them) in one launch: the two need only x, and
// the shared tiles fill the CUs that the routed items' last round leaves idle.
template <int TW>
__global__ __launch_bounds__(kW8Threads) void gate_up_with_shared_kernel(SplitArgs a, GroupedArgs s,
                                                                        int routed_blocks) {
  static_assert(kW8Threads == kThreads, "one workgroup size for both ranges");
  if ((int)blockIdx.x < routed_blocks)
    w8_item<2, ACT_FP8X2>(a, blockIdx.x);
  else
    bf16_gemm_item<2, TW>(s, blockIdx.x - routed_blocks);
}

}  // namespace glm

using namespace glm;

int glm_grouped_tile_rows() { return kSplitTileM; }

// Whether the grouped GEMMs cover these shapes: gate/up K = d, N = I in
// feature tiles of 128 per projection; down K = I, N = d in tiles of 256.
bool glm_grouped_supported(int d, int I) {
  return d % 512 == 0 && I % 256 == 0;
}

static int grouped_launch(hipStream_t stream, GroupedArgs a, int nproj, int max_tiles) {
  // gate/up: 192-row tiles (96 features of each projection) when 256-row
  // tiles would leave the grid below one workgroup per CU
  const bool narrow = nproj == 2 && a.N % 96 == 0 &&
                      (long long)max_tiles * (a.N / (kTileW / 2)) < kNumCUs;
  a.feature_tiles = nproj == 2 ? a.N / (narrow ? 96 : kTileW / 2) : a.N / kTileW;
  // XCD x handles items [x * per, (x + 1) * per) with per <= ceil(max_items / 8),
  // at linear ids x + 8k: the grid must reach 8 * ceil(max_items / 8)
  const long long max_items = (long long)max_tiles * a.feature_tiles;
  const dim3 grid((unsigned)(((max_items + kXcds - 1) / kXcds) * kXcds));
  if (nproj == 2 && narrow)
    hipLaunchKernelGGL((grouped_bf16_gemm_kernel<2, 192>), grid, dim3(kThreads),
                       kStages * (size_t)Bf16Layout<192>::kStageBytes, stream, a);
  else if (nproj == 2)
    hipLaunchKernelGGL((grouped_bf16_gemm_kernel<2, 256>), grid, dim3(kThreads),
                       kStages * (size_t)Bf16Layout<256>::kStageBytes, stream, a);
  else
    hipLaunchKernelGGL((grouped_bf16_gemm_kernel<1, 256>), grid, dim3(kThreads),
                       kStages * (size_t)Bf16Layout<256>::kStageBytes, stream, a);
  GLM_LAUNCH_CHECK("grouped_bf16_gemm_kernel");
  return GLM_OK;
}

size_t glm_act_split_bytes(long long rows, int K) { return SplitLayout(rows, K).total; }

// The block-scaled GEMMs read a split through one buffer resource with 32-bit
// offsets: the whole split must stay below 4 GiB.
bool glm_split_fits(long long rows, int K, int af) {
  return rows >= 0 && K > 0 && SplitLayout(rows, K, af).total <= 0xffffffffull;
}
bool glm_split_fits(long long rows, int K) { return glm_split_fits(rows, K, ACT_FP8X2); }

// bf16 activations [rows][K] -> their split in format af (layout SplitLayout).
static int act_split_launch_as(hipStream_t stream, const uint16_t *x, long long rows, int K,
                               int af, void *split) {
  const long long groups = rows * (K / 32);
  if (groups <= 0) return GLM_OK;
  const SplitLayout L(rows, K, af);
  uint8_t *base = static_cast<uint8_t *>(split);
  const dim3 grid((unsigned)((groups + 255) / 256));
  if (af == ACT_FP8X2)
    hipLaunchKernelGGL(act_split_kernel, dim3((unsigned)((4 * groups + 255) / 256)), dim3(256), 0,
                       stream, x, groups, base,
                       base + L.lo, base + L.shi, base + L.slo);
  else if (af == ACT_FP8FP6)
    hipLaunchKernelGGL(act_split_fp8fp6_kernel, grid, dim3(256), 0, stream, x, groups, K, base,
                       base + L.lo, base + L.shi, base + L.slo);
  else if (af == ACT_FP6X2)
    hipLaunchKernelGGL(act_split_lowp_kernel<ACT_FP6X2>, grid, dim3(256), 0, stream, x, groups, K,
                       base, base + L.lo, base + L.shi, base + L.slo);
  else
    hipLaunchKernelGGL(act_split_lowp_kernel<ACT_FP4>, grid, dim3(256), 0, stream, x, groups, K,
                       base, base, base + L.shi, base + L.shi);
  GLM_LAUNCH_CHECK("act_split_kernel");
  return GLM_OK;
}

// Router weights [E][d] f32 -> their three bf16 parts (wsplit), and x [T][d]
// -> its FP8 hi/lo split, in one launch.
int glm_prefill_split_launch(hipStream_t stream, const float *router_weight, int E, int d,
                             uint16_t *wsplit, const uint16_t *x, int T, void *x_split) {
  const long long nw = (long long)E * d, groups = (long long)T * (d / 32);
  const SplitLayout L(T, d, ACT_FP8X2);
  uint8_t *base = static_cast<uint8_t *>(x_split);
  const int wblocks = (int)((nw + 255) / 256);
  const long long xblocks = (4 * groups + 255) / 256;
  hipLaunchKernelGGL(prefill_split_kernel, dim3((unsigned)(wblocks + xblocks)), dim3(256), 0,
                     stream, router_weight, nw, wsplit, wblocks, x, groups, base, base + L.lo,
                     base + L.shi, base + L.slo);
  GLM_LAUNCH_CHECK("prefill_split_kernel");
  return GLM_OK;
}

int glm_act_split_launch(hipStream_t stream, const uint16_t *x, long long rows, int K,
                         void *split) {
  return act_split_launch_as(stream, x, rows, K, ACT_FP8X2, split);
}

// The eight-wave form runs the gate/up GEMMs (T = 4096: 186.8 against 198.4 us
// and 197 against 210 us, interleaved, on two boxes); the down GEMMs stay on
// sixteen waves, which the eight-wave form did not beat (122 against 121 us).
constexpr int kSplitWavesGateUp = 8, kSplitWavesDown = 16;

template <int NPROJ, int AF>
static void launch_f8f6f4(hipStream_t stream, dim3 grid, const SplitArgs &a) {
  constexpr int waves = NPROJ == 2 ? kSplitWavesGateUp : kSplitWavesDown;
  if constexpr (waves == 8)
    hipLaunchKernelGGL((grouped_f8f6f4_w8_kernel<NPROJ, AF>), grid, dim3(kW8Threads),
                       (size_t)W8Layout<AF>::kBytes, stream, a);
  else
    hipLaunchKernelGGL((grouped_f8f6f4_kernel<NPROJ, AF>), grid, dim3(kSplitThreads),
                       kSplitStages * (size_t)SplitStage<AF>::kBytes, stream, a);
}

static int split_launch(hipStream_t stream, SplitArgs a, int nproj, int max_tiles, int af) {
  a.feature_tiles = a.N / (nproj == 2 ? kSplitTileW / 2 : kSplitTileW);
  a.max_tiles = max_tiles;
  // XCD x handles items [x * per, (x + 1) * per) with per <= ceil(max_items / 8),
  // at linear ids x + 8k: the grid must reach 8 * ceil(max_items / 8)
  const long long max_items = (long long)max_tiles * a.feature_tiles;
  const dim3 grid((unsigned)(((max_items + kXcds - 1) / kXcds) * kXcds));
  if (nproj == 2) {
    if (af == ACT_FP8X2)
      launch_f8f6f4<2, ACT_FP8X2>(stream, grid, a);
    else if (af == ACT_FP6X2)
      launch_f8f6f4<2, ACT_FP6X2>(stream, grid, a);
    else if (af == ACT_FP8FP6)
      launch_f8f6f4<2, ACT_FP8FP6>(stream, grid, a);
    else
      launch_f8f6f4<2, ACT_FP4>(stream, grid, a);
  } else {
    if (af == ACT_FP8X2)
      launch_f8f6f4<1, ACT_FP8X2>(stream, grid, a);
    else if (af == ACT_FP6X2)
      launch_f8f6f4<1, ACT_FP6X2>(stream, grid, a);
    else if (af == ACT_FP8FP6)
      launch_f8f6f4<1, ACT_FP8FP6>(stream, grid, a);
    else
      launch_f8f6f4<1, ACT_FP4>(stream, grid, a);
  }
  GLM_LAUNCH_CHECK("grouped_f8f6f4_kernel");
  return GLM_OK;
}

static void set_split(SplitArgs &a, const void *split, long long rows, int K, int af) {
  const SplitLayout L(rows, K, af);
  const uint8_t *base = static_cast<const uint8_t *>(split);
  a.split_bytes = (uint32_t)L.total;
  a.xhi = base;
  a.xlo = base + L.lo;
  a.xshi = base + L.shi;
  a.xslo = af == ACT_FP4 ? base + L.shi : base + L.slo;
}

// x_split: the split (format af) of the T token rows of x (d columns).
// h_split (ACT_FP8X2 only): when set, the epilogue writes the split of h
// [P][I] instead of h.
static int grouped_gate_up_as(hipStream_t stream, const void *x_split, int T,
                              const int32_t *pair_token, const int4 *tiles,
                              const int32_t *num_tiles, int max_tiles, int d, int I,
                              const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                              const uint8_t *us, uint16_t *h, float limit, void *h_split,
                              long long P, int af) {
  SplitArgs a{};
  set_split(a, x_split, T, d, af);
  a.out_split = static_cast<uint8_t *>(h_split);
  a.out_rows = P;
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
  return split_launch(stream, a, 2, max_tiles, af);
}

int glm_grouped_gate_up_launch(hipStream_t stream, const void *x_split, int T,
                               const int32_t *pair_token, const int4 *tiles,
                               const int32_t *num_tiles, int max_tiles, int d, int I,
                               const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                               const uint8_t *us, uint16_t *h, float limit, void *h_split,
                               long long P) {
  return grouped_gate_up_as(stream, x_split, T, pair_token, tiles, num_tiles, max_tiles, d, I, gw,
                            gs, uw, us, h, limit, h_split, P, ACT_FP8X2);
}

// h_split: the split (format af) of the P sorted rows of h (I columns).
static int grouped_down_as(hipStream_t stream, const void *h_split, long long P,
                           const int4 *tiles, const int32_t *num_tiles, int max_tiles, int I,
                           int d, const uint8_t *dw, const uint8_t *ds, uint16_t *y, int af) {
  SplitArgs a{};
  set_split(a, h_split, P, I, af);
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
  return split_launch(stream, a, 1, max_tiles, af);
}

int glm_grouped_down_launch(hipStream_t stream, const void *h_split, long long P,
                            const int4 *tiles, const int32_t *num_tiles, int max_tiles, int I,
                            int d, const uint8_t *dw, const uint8_t *ds, uint16_t *y) {
  return grouped_down_as(stream, h_split, P, tiles, num_tiles, max_tiles, I, d, dw, ds, y,
                         ACT_FP8X2);
}

// Dense bf16 SwiGLU MLP over T token rows (the shared expert at many tokens):
// h = limited_swiglu(bf16(x Wg^T), bf16(x Wu^T)); out = bf16(h Wd^T).
// The layer's routed gate/up (FP8 split of x; the epilogue writes h's split)
// and the bf16 shared expert's gate/up (x [T][d] -> shared_h [T][Is], dense
// mode) in one launch, gate_up_with_shared_kernel: the routed workgroups as
// split_launch grids them, then the shared ones as grouped_launch does (192- or
// 256-row weight tiles).  The shared down follows with glm_grouped_dense_down_launch.
int glm_grouped_gate_up_shared_launch(hipStream_t stream, const void *x_split, int T,
                                      const int32_t *pair_token, const int4 *tiles,
                                      const int32_t *num_tiles, int max_tiles, int d, int I,
                                      const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                                      const uint8_t *us, uint16_t *h, float limit, void *h_split,
                                      long long P, const uint16_t *x, int Is, const uint16_t *sgw,
                                      const uint16_t *suw, uint16_t *shared_h) {
  SplitArgs a{};
  set_split(a, x_split, T, d, ACT_FP8X2);
  a.out_split = static_cast<uint8_t *>(h_split);
  a.out_rows = P;
  a.act_index = pair_token;
  a.tiles = tiles;
  a.num_tiles = num_tiles;
  a.max_tiles = max_tiles;
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
  a.feature_tiles = a.N / (kSplitTileW / 2);
  const long long r_items = (long long)max_tiles * a.feature_tiles;
  const long long routed_blocks = (r_items + kXcds - 1) / kXcds * kXcds;
  GroupedArgs sh{};
  sh.act = x;
  sh.dense_rows = T;
  sh.w[0] = reinterpret_cast<const uint8_t *>(sgw);
  sh.w[1] = reinterpret_cast<const uint8_t *>(suw);
  sh.N = Is;
  sh.K = d;
  sh.out = shared_h;
  sh.limit = glm_limit_bf16(limit);
  const int stiles = (T + kTileM - 1) / kTileM;
  const bool narrow = Is % 96 == 0 && (long long)stiles * (Is / (kTileW / 2)) < kNumCUs;
  sh.feature_tiles = Is / (narrow ? 96 : kTileW / 2);
  const long long s_items = (long long)stiles * sh.feature_tiles;
  const long long shared_blocks = (s_items + kXcds - 1) / kXcds * kXcds;
  const dim3 grid((unsigned)(routed_blocks + shared_blocks));
  constexpr size_t kW8 = W8Layout<ACT_FP8X2>::kBytes;
  if (narrow) {
    constexpr size_t kB = kStages * (size_t)Bf16Layout<192>::kStageBytes;
    hipLaunchKernelGGL((gate_up_with_shared_kernel<192>), grid, dim3(kW8Threads), kW8 > kB ? kW8 : kB,
                       stream, a, sh, (int)routed_blocks);
  } else {
    constexpr size_t kB = kStages * (size_t)Bf16Layout<256>::kStageBytes;
    hipLaunchKernelGGL((gate_up_with_shared_kernel<256>), grid, dim3(kW8Threads), kW8 > kB ? kW8 : kB,
                       stream, a, sh, (int)routed_blocks);
  }
  GLM_LAUNCH_CHECK("gate_up_with_shared_kernel");
  return GLM_OK;
}

// The bf16 shared expert's down GEMM alone (dense mode): h [T][Is] -> out [T][d].
int glm_grouped_dense_down_launch(hipStream_t stream, const uint16_t *h, int T, int Is, int d,
                                  const uint16_t *dw, uint16_t *out) {
  GroupedArgs b{};
  b.act = h;
  b.dense_rows = T;
  b.w[0] = b.w[1] = reinterpret_cast<const uint8_t *>(dw);
  b.N = d;
  b.K = Is;
  b.out = out;
  return grouped_launch(stream, b, 1, (T + kTileM - 1) / kTileM);
}

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
  int rc = grouped_launch(stream, a, 2, tiles);
  if (rc) return rc;
  GroupedArgs b{};
  b.act = h;
  b.dense_rows = T;
  b.w[0] = b.w[1] = reinterpret_cast<const uint8_t *>(dw);
  b.N = d;
  b.K = I;
  b.out = out;
  return grouped_launch(stream, b, 1, tiles);
}

bool glm_grouped_supported(int d, int I);

static bool act_format_ok(int af) {
  return af == ACT_FP8X2 || af == ACT_FP6X2 || af == ACT_FP4 || af == ACT_FP8FP6;
}

extern "C" size_t glm_act_split_bytes_fmt(int rows, int K, int act_format) {
  if (rows < 0 || K <= 0 || K % 32 != 0 || !act_format_ok(act_format)) return 0;
  // E2M3 rows are stored in whole 128-element chunks
  if ((act_format == ACT_FP6X2 || act_format == ACT_FP8FP6) && K % 128 != 0) return 0;
  return SplitLayout((long long)rows, K, act_format).total;
}

extern "C" size_t glm_act_split_bytes(int rows, int K) {
  return glm_act_split_bytes_fmt(rows, K, ACT_FP8X2);
}

extern "C" int glm_act_split(void *stream, const uint16_t *x, int rows, int K, int act_format,
                             void *split) {
  glm::clear_error();
  GLM_REQUIRE(x && split, GLM_ERR_INVALID_ARGUMENT, "act_split: null pointer argument");
  GLM_REQUIRE(act_format_ok(act_format), GLM_ERR_INVALID_ARGUMENT,
              "act_split: unknown act_format %d", act_format);
  GLM_REQUIRE(rows >= 0 && K > 0 && K % 32 == 0, GLM_ERR_INVALID_ARGUMENT,
              "act_split: needs rows >= 0 and K %% 32 == 0 (rows=%d K=%d)", rows, K);
  GLM_REQUIRE((act_format != ACT_FP6X2 && act_format != ACT_FP8FP6) || K % 128 == 0,
              GLM_ERR_UNSUPPORTED_SHAPE, "act_split: an E2M3 term needs K %% 128 == 0 (K=%d)", K);
  GLM_REQUIRE(glm_aligned16({x, split}), GLM_ERR_INVALID_ARGUMENT,
              "act_split: buffers must be 16-byte aligned");
  return act_split_launch_as((hipStream_t)stream, x, rows, K, act_format, split);
}

extern "C" int glm_act_split_fp8(void *stream, const uint16_t *x, int rows, int K, void *split) {
  return glm_act_split(stream, x, rows, K, ACT_FP8X2, split);
}

extern "C" int glm_expert_gate_up_grouped_fmt(void *stream, int act_format, const void *x_split,
                                              int T, int d, int I, const uint8_t *gate_packed,
                                              const uint8_t *gate_scales,
                                              const uint8_t *up_packed, const uint8_t *up_scales,
                                              const int32_t *pair_token, const int32_t *tiles,
                                              const int32_t *num_tiles, int max_tiles,
                                              float swiglu_limit, uint16_t *h) {
  glm::clear_error();
  GLM_REQUIRE(x_split && gate_packed && gate_scales && up_packed && up_scales && pair_token &&
                  tiles && num_tiles && h,
              GLM_ERR_INVALID_ARGUMENT, "expert_gate_up_grouped: null pointer argument");
  GLM_REQUIRE(act_format_ok(act_format), GLM_ERR_INVALID_ARGUMENT,
              "expert_gate_up_grouped: unknown act_format %d", act_format);
  GLM_REQUIRE(max_tiles >= 0 && T >= 0, GLM_ERR_INVALID_ARGUMENT,
              "expert_gate_up_grouped: max_tiles < 0 or T < 0");
  GLM_REQUIRE(glm_grouped_supported(d, I), GLM_ERR_UNSUPPORTED_SHAPE,
              "expert_gate_up_grouped: needs d %% 512 == 0 and I %% 256 == 0 (d=%d I=%d)", d, I);
  GLM_REQUIRE(glm_aligned16({x_split, gate_packed, up_packed, tiles, h}),
              GLM_ERR_INVALID_ARGUMENT, "expert_gate_up_grouped: buffers must be 16-byte aligned");
  GLM_REQUIRE(glm_split_fits(T, d, act_format), GLM_ERR_UNSUPPORTED_SHAPE,
              "expert_gate_up_grouped: the split of %d x %d activations exceeds 4 GiB", T, d);
  if (max_tiles == 0 || T == 0) return GLM_OK;
  return grouped_gate_up_as((hipStream_t)stream, x_split, T, pair_token,
                            reinterpret_cast<const int4 *>(tiles), num_tiles, max_tiles, d, I,
                            gate_packed, gate_scales, up_packed, up_scales, h, swiglu_limit,
                            nullptr, 0, act_format);
}

extern "C" int glm_expert_gate_up_grouped(void *stream, const void *x_split, int T, int d, int I,
                                          const uint8_t *gate_packed, const uint8_t *gate_scales,
                                          const uint8_t *up_packed, const uint8_t *up_scales,
                                          const int32_t *pair_token, const int32_t *tiles,
                                          const int32_t *num_tiles, int max_tiles,
                                          float swiglu_limit, uint16_t *h) {
  return glm_expert_gate_up_grouped_fmt(stream, ACT_FP8X2, x_split, T, d, I, gate_packed,
                                        gate_scales, up_packed, up_scales, pair_token, tiles,
                                        num_tiles, max_tiles, swiglu_limit, h);
}

extern "C" int glm_expert_down_grouped_fmt(void *stream, int act_format, const void *h_split,
                                           int P, int I, int d, const uint8_t *down_packed,
                                           const uint8_t *down_scales, const int32_t *tiles,
                                           const int32_t *num_tiles, int max_tiles, uint16_t *y) {
  glm::clear_error();
  GLM_REQUIRE(h_split && down_packed && down_scales && tiles && num_tiles && y,
              GLM_ERR_INVALID_ARGUMENT, "expert_down_grouped: null pointer argument");
  GLM_REQUIRE(act_format_ok(act_format), GLM_ERR_INVALID_ARGUMENT,
              "expert_down_grouped: unknown act_format %d", act_format);
  GLM_REQUIRE(max_tiles >= 0 && P >= 0, GLM_ERR_INVALID_ARGUMENT,
              "expert_down_grouped: max_tiles < 0 or P < 0");
  GLM_REQUIRE(glm_grouped_supported(d, I), GLM_ERR_UNSUPPORTED_SHAPE,
              "expert_down_grouped: needs d %% 512 == 0 and I %% 256 == 0 (d=%d I=%d)", d, I);
  GLM_REQUIRE(glm_aligned16({h_split, down_packed, tiles, y}), GLM_ERR_INVALID_ARGUMENT,
              "expert_down_grouped: buffers must be 16-byte aligned");
  GLM_REQUIRE(glm_split_fits(P, I, act_format), GLM_ERR_UNSUPPORTED_SHAPE,
              "expert_down_grouped: the split of %d x %d activations exceeds 4 GiB", P, I);
  if (max_tiles == 0 || P == 0) return GLM_OK;
  return grouped_down_as((hipStream_t)stream, h_split, P, reinterpret_cast<const int4 *>(tiles),
                         num_tiles, max_tiles, I, d, down_packed, down_scales, y, act_format);
}

extern "C" int glm_expert_down_grouped(void *stream, const void *h_split, int P, int I, int d,
                                       const uint8_t *down_packed, const uint8_t *down_scales,
                                       const int32_t *tiles, const int32_t *num_tiles,
                                       int max_tiles, uint16_t *y) {
  return glm_expert_down_grouped_fmt(stream, ACT_FP8X2, h_split, P, I, d, down_packed,
                                     down_scales, tiles, num_tiles, max_tiles, y);
}
