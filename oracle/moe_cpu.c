/*
 * CPU restatement of livglm's routed-MoE layer -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain C + OpenMP twin of oracle/moe_oracle.py, used (1) by the tests to
 * cross-check the numpy oracle at sizes numpy is slow on and (2) as the
 * benchmark's CPU baseline ("CPU restatement (not MLX)": the reference's own
 * CPU path is MLX, which is unavailable).  It is never part of the product.
 *
 * Follows the reference: router moe.py:36-63; routed SwitchGLU
 * expert_ssd.py:159-188 with limited_swiglu expert_ssd.py:103-107; shared
 * DenseMLP layers.py:160-171; merge moe.py:198-201.  Rounding points: f32
 * accumulation (fixed 8-lane partial sums per 32-element group), bf16 rounding
 * of every projection output and of each SwiGLU step, f32 merge in sequential
 * top-k order.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

static const float E2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                               -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

static inline float e8m0(uint8_t e) {
  if (e == 255) return NAN;
  return ldexpf(1.0f, (int)e - 127);
}

static inline float sigmoid_f32(float x) {
  float y = 1.0f / (1.0f + expf(fabsf(x)));
  return x < 0.0f ? y : 1.0f - y;
}

/* limited_swiglu (expert_ssd.py:103-107); a NaN g or u passes through the
 * clamps, as through mx.minimum / mx.clip and numpy's minimum / clip. */
static inline float swiglu(float g, float u, float L) {
  if (L > 0.0f) {
    g = g > L ? L : g;
    u = u < -L ? -L : (u > L ? L : u);
  }
  float s = bf16_round(sigmoid_f32(g));
  float a = bf16_round(g * s);
  return bf16_round(a * u);
}

/* One MXFP4 row (K/2 packed bytes, K/32 scales) dotted with an f32 vector. */
static float dot_mxfp4(const uint8_t *packed, const uint8_t *scales, const float *x, int K) {
  float total = 0.0f;
  for (int g = 0; g < K / 32; ++g) {
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint8_t *p = packed + g * 16;
    const float *xv = x + g * 32;
    for (int b = 0; b < 16; ++b) {
      lane[(2 * b) & 7] += E2M1[p[b] & 15] * xv[2 * b];
      lane[(2 * b + 1) & 7] += E2M1[p[b] >> 4] * xv[2 * b + 1];
    }
    float part = ((lane[0] + lane[1]) + (lane[2] + lane[3])) + ((lane[4] + lane[5]) + (lane[6] + lane[7]));
    total += part * e8m0(scales[g]);
  }
  return total;
}

static float dot_bf16(const uint16_t *w, const float *x, int K) {
  float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = 0; i < K; ++i) lane[i & 7] += bf16_to_f32(w[i]) * x[i];
  return ((lane[0] + lane[1]) + (lane[2] + lane[3])) + ((lane[4] + lane[5]) + (lane[6] + lane[7]));
}

int moe_cpu_threads(void) { return omp_get_max_threads(); }

static int better(float v1, int i1, float v2, int i2) { return v1 > v2 || (v1 == v2 && i1 > i2); }

/* Router for one token: logits/scores, group mask, top-k ascending. */
static void route_token(const float *xf, int d, const float *rw, const float *rb, int E, int k,
                        int n_group, int topk_group, int norm, float scale, float *w_out,
                        uint32_t *idx_out, float *work) {
  float *score = work, *choice = work + E;
  for (int e = 0; e < E; ++e) {
    double acc = 0.0;
    const float *row = rw + (size_t)e * d;
    for (int i = 0; i < d; ++i) acc += (double)xf[i] * (double)row[i];
    float l = (float)acc;
    score[e] = sigmoid_f32(l);
    choice[e] = score[e] + rb[e];
    if (choice[e] != choice[e]) choice[e] = -INFINITY; /* NaN ranks as -inf */
  }
  if (n_group > 1) {
    int per = E / n_group;
    float gs[1024];
    for (int g = 0; g < n_group; ++g) {
      float t1 = -INFINITY, t2 = -INFINITY;
      for (int q = 0; q < per; ++q) {
        float v = choice[g * per + q];
        if (v > t1) {
          t2 = t1;
          t1 = v;
        } else if (v > t2) {
          t2 = v;
        }
      }
      gs[g] = t2 + t1;
    }
    for (int g = 0; g < n_group; ++g) {
      int rank = 0;
      for (int h = 0; h < n_group; ++h) rank += better(gs[h], h, gs[g], g);
      if (rank >= topk_group)
        for (int q = 0; q < per; ++q) choice[g * per + q] = -INFINITY;
    }
  }
  unsigned char taken[1024];
  memset(taken, 0, sizeof(taken));
  for (int r = 0; r < k; ++r) {
    int bi = -1;
    for (int e = 0; e < E; ++e)
      if (!taken[e] && (bi < 0 || better(choice[e], e, choice[bi], bi))) bi = e;
    taken[bi] = 1;
    idx_out[k - 1 - r] = (uint32_t)bi;
    w_out[k - 1 - r] = score[bi];
  }
  float total = 0.0f;
  if (norm)
    for (int j = 0; j < k; ++j) total += w_out[j];
  for (int j = 0; j < k; ++j) {
    float v = w_out[j];
    if (norm) v = v / (total + 1e-20f);
    w_out[j] = v * scale;
  }
}

/* Whole layer on host buffers; arguments mirror glm_moe_forward (bf16 shared
 * expert).  Returns 0, or -1 on a bad argument / allocation failure. */
int moe_cpu_layer(const uint16_t *x, int T, int d, const float *rw, const float *rb, int E, int k,
                  int n_group, int topk_group, int norm, float scale, int I, const uint8_t *gw,
                  const uint8_t *gs, const uint8_t *uw, const uint8_t *us, const uint8_t *dw,
                  const uint8_t *ds, int Is, const uint16_t *sg, const uint16_t *su,
                  const uint16_t *sd, float limit, float *out, float *w_out, uint32_t *idx_out) {
  if (T < 0 || d % 32 || I % 32 || E < 1 || E > 1024 || k < 1 || k > E) return -1;
  const float L = bf16_round(limit);
  const size_t P = (size_t)T * k;
  float *xf = malloc(sizeof(float) * (size_t)T * d);
  float *h = malloc(sizeof(float) * P * I);
  float *y = malloc(sizeof(float) * P * d);
  int *cnt = calloc((size_t)E + 1, sizeof(int));
  int *pairs = malloc(sizeof(int) * (P ? P : 1));
  float *shared = Is > 0 ? malloc(sizeof(float) * (size_t)T * d) : NULL;
  float *hs = Is > 0 ? malloc(sizeof(float) * (size_t)T * Is) : NULL;
  if (!xf || !h || !y || !cnt || !pairs || (Is > 0 && (!shared || !hs))) {
    free(xf), free(h), free(y), free(cnt), free(pairs), free(shared), free(hs);
    return -1;
  }
  for (size_t i = 0; i < (size_t)T * d; ++i) xf[i] = bf16_to_f32(x[i]);

#pragma omp parallel
  {
    float *work = malloc(sizeof(float) * 2 * E);
#pragma omp for schedule(static)
    for (int t = 0; t < T; ++t)
      route_token(xf + (size_t)t * d, d, rw, rb, E, k, n_group, topk_group, norm, scale,
                  w_out + (size_t)t * k, idx_out + (size_t)t * k, work);
    free(work);
  }

  /* group pairs by expert (stable), so each expert's rows are read once */
  for (size_t p = 0; p < P; ++p) cnt[idx_out[p] + 1]++;
  for (int e = 0; e < E; ++e) cnt[e + 1] += cnt[e];
  {
    int *fill = malloc(sizeof(int) * E);
    memcpy(fill, cnt, sizeof(int) * E);
    for (size_t p = 0; p < P; ++p) pairs[fill[idx_out[p]]++] = (int)p;
    free(fill);
  }

  const size_t gate_row = (size_t)d / 2, gate_srow = (size_t)d / 32;
  const size_t down_row = (size_t)I / 2, down_srow = (size_t)I / 32;
#pragma omp parallel for collapse(2) schedule(dynamic, 16)
  for (int e = 0; e < E; ++e)
    for (int i = 0; i < I; ++i) {
      const int n = cnt[e + 1] - cnt[e];
      if (n == 0) continue;
      const size_t r = (size_t)e * I + i;
      for (int q = 0; q < n; ++q) {
        const int p = pairs[cnt[e] + q];
        const float *xv = xf + (size_t)(p / k) * d;
        float g = bf16_round(dot_mxfp4(gw + r * gate_row, gs + r * gate_srow, xv, d));
        float u = bf16_round(dot_mxfp4(uw + r * gate_row, us + r * gate_srow, xv, d));
        h[(size_t)p * I + i] = swiglu(g, u, L);
      }
    }
#pragma omp parallel for collapse(2) schedule(dynamic, 16)
  for (int e = 0; e < E; ++e)
    for (int c = 0; c < d; ++c) {
      const int n = cnt[e + 1] - cnt[e];
      if (n == 0) continue;
      const size_t r = (size_t)e * d + c;
      for (int q = 0; q < n; ++q) {
        const int p = pairs[cnt[e] + q];
        y[(size_t)p * d + c] =
            bf16_round(dot_mxfp4(dw + r * down_row, ds + r * down_srow, h + (size_t)p * I, I));
      }
    }
  if (Is > 0) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < T; ++t)
      for (int i = 0; i < Is; ++i) {
        const float *xv = xf + (size_t)t * d;
        float g = bf16_round(dot_bf16(sg + (size_t)i * d, xv, d));
        float u = bf16_round(dot_bf16(su + (size_t)i * d, xv, d));
        hs[(size_t)t * Is + i] = swiglu(g, u, L);
      }
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < T; ++t)
      for (int c = 0; c < d; ++c)
        shared[(size_t)t * d + c] = bf16_round(dot_bf16(sd + (size_t)c * Is, hs + (size_t)t * Is, Is));
  }
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t)
    for (int c = 0; c < d; ++c) {
      float acc = 0.0f;
      for (int j = 0; j < k; ++j) {
        float prod = y[((size_t)t * k + j) * d + c] * w_out[(size_t)t * k + j];
        acc = acc + prod;
      }
      if (shared) acc = acc + shared[(size_t)t * d + c];
      out[(size_t)t * d + c] = acc;
    }
  free(xf), free(h), free(y), free(cnt), free(pairs), free(shared), free(hs);
  return 0;
}

/* E4M3FN element value (fp8.py:13-30): bias 7, subnormals below 2^-6,
 * 0x7F / 0xFF NaN. */
static float e4m3fn(uint8_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7) v = NAN;
  else if (e == 0) v = ldexpf((float)m / 8.0f, -6);
  else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return (c & 0x80) ? -v : v;
}

/* Resident MXFP8 linear y = bf16(x . deq(W)^T) (layers.py:56-65): codes
 * [out][in] E4M3FN, scales [out][in/32] E8M0, x and y bf16. */
int moe_cpu_linear_mxfp8(const uint16_t *x, int T, int in_dims, const uint8_t *codes,
                         const uint8_t *scales, int out_dims, uint16_t *y) {
  if (T < 0 || in_dims % 32 || out_dims < 1) return -1;
  float lut[256];
  for (int c = 0; c < 256; ++c) lut[c] = e4m3fn((uint8_t)c);
  float *xf = (float *)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1) * in_dims);
  for (size_t i = 0; i < (size_t)T * in_dims; ++i) xf[i] = bf16_to_f32(x[i]);
#pragma omp parallel for collapse(2) schedule(static)
  for (int t = 0; t < T; ++t)
    for (int o = 0; o < out_dims; ++o) {
      const uint8_t *row = codes + (size_t)o * in_dims;
      const float *xv = xf + (size_t)t * in_dims;
      float total = 0.0f;
      for (int g = 0; g < in_dims / 32; ++g) {
        float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int i = 0; i < 32; ++i) lane[i & 7] += lut[row[g * 32 + i]] * xv[g * 32 + i];
        float part = ((lane[0] + lane[1]) + (lane[2] + lane[3])) + ((lane[4] + lane[5]) + (lane[6] + lane[7]));
        total += part * e8m0(scales[(size_t)o * (in_dims / 32) + g]);
      }
      y[(size_t)t * out_dims + o] = f32_to_bf16(total);
    }
  free(xf);
  return 0;
}
