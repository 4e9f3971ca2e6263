// Top-k expert selection of one token by one wave (TopKRouter.__call__,
// moe.py:39-62), shared by the router kernels and the decode-layer kernels.
#pragma once

#include "glm_common.h"

namespace glm {

// Lexicographic "better" for (value, index): larger value; on a tie the
// larger index (a stable ascending argsort puts it last, moe.py:33-34).
__device__ __forceinline__ bool better(float v1, int i1, float v2, int i2) {
  return v1 > v2 || (v1 == v2 && i1 > i2);
}

// Orders LDS traffic between the lanes of one wave.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, true);
}

// Maximum of an int over the wave, left in every lane: DPP within each row
// of 16 lanes (quad swaps, then row rotations by 4 and 8), then across the
// rows through gfx950's row swaps -- all vector ALU, no scalar round trip.
__device__ __forceinline__ int wave_max_i32(int v) {
  v = max(v, dpp_i32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_i32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_i32<0x124>(v));  // row_ror:4
  v = max(v, dpp_i32<0x128>(v));  // row_ror:8
  const auto s = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  v = max((int)s[0], (int)s[1]);  // rows 0|1 and 2|3
  const auto t = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return max((int)t[0], (int)t[1]);
}

// Signed-int key with the order of a non-NaN float (-0 must be folded to +0
// first so that equal floats have equal keys).
__device__ __forceinline__ int order_key(float v) {
  const int b = __float_as_int(v);
  return b >= 0 ? b : b ^ 0x7fffffff;
}

// Top-k selection of one token by one wave (moe.py:39-62).  Lane l holds
// experts l + 64i; k rounds of a DPP wave maximum over sortable keys pick the
// experts best first.  Lanes j < k write column j of the weights and indices
// (skipped where w_out / i_out are null) and of pair_idx.
// `scratch` is this wave's LDS area (>= 64*EPL + 256 words).
template <int EPL>
__device__ void select_token(const float *logits_row, const float *bias, int E, int k,
                             int n_group, int topk_group, int norm, float scale, float *w_out,
                             uint32_t *i_out, int *pair_idx, float *scratch, int lane) {
  float score[EPL], choice[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    score[i] = 0.0f;
    choice[i] = -INFINITY;
    if (e < E) {
      score[i] = sigmoid_f32(logits_row[e]);
      choice[i] = score[i] + bias[e];
    }
  }
  float *s_choice = scratch;            // [64*EPL]
  float *s_g = scratch + 64 * EPL;      // [64] group scores
  int *s_keep = (int *)(s_g + 64);      // [64]
  int *s_isel = s_keep + 64;            // [64]
  float *s_wsel = (float *)(s_isel + 64);  // [64]
  if (n_group > 1) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) s_choice[lane + 64 * i] = choice[i];
    wave_lds_sync();
    const int per = E / n_group;
    if (lane < n_group) {
      float t1 = -INFINITY, t2 = -INFINITY;
      for (int qq = 0; qq < per; ++qq) {
        const float v = s_choice[lane * per + qq];
        if (v > t1) {
          t2 = t1;
          t1 = v;
        } else if (v > t2) {
          t2 = v;
        }
      }
      s_g[lane] = t2 + t1;
    }
    wave_lds_sync();
    if (lane < n_group) {
      const float mine = s_g[lane];
      int rank = 0;
      for (int g = 0; g < n_group; ++g) rank += better(s_g[g], g, mine, lane) ? 1 : 0;
      s_keep[lane] = rank < topk_group;
    }
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !s_keep[e / per]) choice[i] = -INFINITY;
    }
  }
  // k rounds: the wave maximum of the remaining choices, then, among the
  // experts holding it, the largest index (a stable ascending argsort ranks
  // equal values by index, moe.py:33-34).  The winner of round r lands in
  // ascending column k-1-r and drops out.  NaN choices rank as -inf; absent
  // and chosen experts hold INT_MIN, below every real key.
  int key[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const float c = choice[i] != choice[i] ? -INFINITY : choice[i] + 0.0f;  // NaN -> -inf, -0 -> +0
    key[i] = lane + 64 * i < E ? order_key(c) : INT_MIN;
  }
  // Lane k-1-r keeps round r's expert and score.  The winner is almost always
  // the only expert holding the maximum: one ballot names its lane, whose
  // highest slot holding it is the slot.  On a tie the highest such slot over
  // the wave wins, then the highest lane holding it there.
  int my_idx = 0;
  float my_w = 0.0f;
  for (int r = 0; r < k; ++r) {
    int m = key[0];
#pragma unroll
    for (int i = 1; i < EPL; ++i) m = max(m, key[i]);
    const int best = wave_max_i32(m);
    int slot_l = -1;  // this lane's highest slot holding the maximum
    float sc_l = 0.0f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const bool hit = key[i] == best;
      slot_l = hit ? i : slot_l;
      sc_l = hit ? score[i] : sc_l;
    }
    const unsigned long long bal = __ballot(slot_l >= 0);
    int wl, slot;
    if (__popcll(bal) == 1) {
      wl = __ffsll((long long)bal) - 1;
      slot = __builtin_amdgcn_readlane(slot_l, wl);
    } else {
      slot = wave_max_i32(slot_l);
      wl = 63 - __clzll((long long)__ballot(slot_l == slot));
    }
    const float wsc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc_l), wl));
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (lane == wl && i == slot) key[i] = INT_MIN;
    const bool mine = lane == k - 1 - r;
    my_idx = mine ? wl + 64 * slot : my_idx;
    my_w = mine ? wsc : my_w;
  }
  if (lane < k) {
    s_isel[lane] = my_idx;
    s_wsel[lane] = my_w;
  }
  wave_lds_sync();
  // every lane forms the same sequential sum; lane j < k writes column j
  float total = 0.0f;
  if (norm)
    for (int j = 0; j < k; ++j) total += s_wsel[j];
  if (lane < k) {
    float wj = s_wsel[lane];
    if (norm) wj = wj / (total + 1e-20f);
    if (w_out != nullptr) w_out[lane] = wj * scale;
    if (i_out != nullptr) i_out[lane] = (uint32_t)s_isel[lane];
    pair_idx[lane] = s_isel[lane];
  }
  wave_lds_sync();
}

}  // namespace glm
