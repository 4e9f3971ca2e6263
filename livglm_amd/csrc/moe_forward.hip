// Whole routed-MoE layer (ExpertSSDMoE._call_impl, moe.py:123-201) on one
// stream, plus the library's error plumbing and version query.
#include <mutex>
#include <string>

#include "glm_common.h"
#include "scalex_tile.h"

// ---------------------------------------------------------------- errors

namespace glm {

static thread_local std::string g_last_error;

void set_error(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

}  // namespace glm

extern "C" int glm_abi_version(void) { return GLM_ABI_VERSION; }

extern "C" const char *glm_last_error(void) { return glm::g_last_error.c_str(); }

// ---------------------------------------------------------------- launchers from other units

int glm_router_validate(const void *x, int T, int d, const void *weight, const void *bias, int E,
                        int k, int n_group, int topk_group, const void *weights,
                        const void *indices);
int glm_router_launch(hipStream_t stream, const uint16_t *x, int T, int d, const float *weight,
                      const float *bias, int E, int k, int n_group, int topk_group, int norm,
                      float scale, float *logits, float *weights, uint32_t *indices,
                      uint16_t *wsplit, bool wsplit_ready);
bool glm_router_split_supported(int T, int d);
int glm_prefill_split_launch(hipStream_t stream, const float *router_weight, int E, int d,
                             uint16_t *wsplit, const uint16_t *x, int T, void *x_split);
size_t glm_router_split_bytes(int E, int d);
int glm_dispatch_launch(hipStream_t stream, const uint32_t *indices, int T, int k, int E,
                        int32_t *counts, int32_t *offsets, int32_t *perm, int32_t *inv,
                        int32_t *pair_token, int32_t *active, int32_t *num_active, int4 *work,
                        int32_t *status, int tile_rows, int4 *tiles, int32_t *num_tiles,
                        int32_t *chunk_scratch);
size_t glm_dispatch_chunk_ints(long long P, int E);
int glm_grouped_tile_rows();
bool glm_grouped_supported(int d, int I);
bool glm_split_fits(long long rows, int K);
size_t glm_act_split_bytes(long long rows, int K);
int glm_act_split_launch(hipStream_t stream, const uint16_t *x, long long rows, int K,
                         void *split);
int glm_grouped_gate_up_launch(hipStream_t stream, const void *x_split, int T,
                               const int32_t *pair_token, const int4 *tiles,
                               const int32_t *num_tiles, int max_tiles, int d, int I,
                               const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                               const uint8_t *us, uint16_t *h, float limit, void *h_split,
                               long long P);
int glm_grouped_down_launch(hipStream_t stream, const void *h_split, long long P,
                            const int4 *tiles, const int32_t *num_tiles, int max_tiles, int I,
                            int d, const uint8_t *dw, const uint8_t *ds, uint16_t *y);
int glm_gate_up_launch(hipStream_t stream, const uint16_t *x, int T, int d, int I, int E, int k,
                       const uint8_t *gw, const uint8_t *gs, const uint8_t *uw, const uint8_t *us,
                       const int32_t *pair_token, const int4 *work, float limit, uint16_t *h);
int glm_down_launch(hipStream_t stream, const uint16_t *h, int T, int k, int I, int d, int E,
                    const uint8_t *dw, const uint8_t *ds, const int4 *work, uint16_t *y);
int glm_mlp_launch(hipStream_t stream, const uint16_t *x, int T, int d, int I, int fmt,
                   const void *gw, const uint8_t *gs, const void *uw, const uint8_t *us,
                   const void *dw, const uint8_t *ds, float limit, uint16_t *h, uint16_t *out);
bool glm_grouped_dense_mlp_supported(int T, int d, int I, int fmt);
int glm_grouped_gate_up_shared_launch(hipStream_t stream, const void *x_split, int T,
                                      const int32_t *pair_token, const int4 *tiles,
                                      const int32_t *num_tiles, int max_tiles, int d, int I,
                                      const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                                      const uint8_t *us, uint16_t *h, float limit, void *h_split,
                                      long long P, const uint16_t *x, int Is, const uint16_t *sgw,
                                      const uint16_t *suw, uint16_t *shared_h);
int glm_grouped_dense_down_launch(hipStream_t stream, const uint16_t *h, int T, int Is, int d,
                                  const uint16_t *dw, uint16_t *out);
int glm_combine_launch(hipStream_t stream, const uint16_t *y, const int32_t *inv, const float *w,
                       const uint16_t *shared, int T, int k, int d, float *out);
bool glm_decode_path_supported(int T, int d, int E, int k, int I, int Is);
bool glm_pair_path_supported(int T, int d, int E, int k, int I, int Is);
int glm_pair_path_launch(hipStream_t stream, const uint16_t *x, int T, int d, const float *w,
                         const float *bias, int E, int k, int n_group, int topk_group, int norm,
                         float scale, float *logits, float *weights, uint32_t *indices, int I,
                         const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                         const uint8_t *us, const uint8_t *dw, const uint8_t *ds,
                         const uint16_t *sg, const uint16_t *su, const uint16_t *sd, int Is,
                         float *gp, float *up, uint16_t *hs, float *yp,
                         const uint16_t *shared_ready, uint16_t *h, float limit, float *out,
                         const glm::HcFuse *hc, const uint8_t *sx, long long sx_stride);
int glm_route_decode_launch(hipStream_t stream, const uint16_t *x, int T, int d, const float *w,
                            const float *bias, int E, int k, int n_group, int topk_group,
                            int norm, float scale, float *logits, float *weights,
                            uint32_t *indices, int32_t *counts, int32_t *offsets, int32_t *perm,
                            int32_t *inv, int32_t *pair_token, int32_t *active,
                            int32_t *num_active, int32_t *status, int4 *work,
                            const uint16_t *sg, const uint16_t *su, const uint16_t *sd, int Is,
                            float *gp, float *up, uint16_t *hs, float *yp, float limit);
int glm_decode_gate_up_launch(hipStream_t stream, const uint16_t *x, int T, int d, int I, int E,
                              int k, const uint8_t *gw, const uint8_t *gs, const uint8_t *uw,
                              const uint8_t *us, const int32_t *pair_token, const int4 *work,
                              uint16_t *h, float limit, const uint16_t *sg, const uint16_t *su,
                              int Is, uint16_t *hs);
int glm_decode_down_launch(hipStream_t stream, const uint16_t *h, int T, int k, int I, int d,
                           int E, const uint8_t *dw, const uint8_t *ds, const int4 *work,
                           uint16_t *y, const uint16_t *sd, int Is, uint16_t *hs, float *yp);
bool glm_decode_shared_in_experts(int T, int d);
int glm_combine_parts_launch(hipStream_t stream, const uint16_t *y, const int32_t *inv,
                             const float *w, const uint16_t *shared, const float *shared_parts,
                             int nparts, int T, int k, int d, float *out);
int glm_decode_shared_skq(int T, int d);
int glm_decode_shared_skd(int Is);
int glm_fill_zero_launch(hipStream_t stream, void *p, size_t bytes);

// ---------------------------------------------------------------- workspace

namespace {

constexpr size_t kAlign = 256;

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Workspace {
  float *logits;
  float *weights;
  uint32_t *indices;
  int32_t *counts;
  int32_t *offsets;
  int32_t *active;
  int32_t *num_active;
  int32_t *status;
  int32_t *perm;
  int32_t *inv;
  int32_t *pair_token;
  uint16_t *h;
  uint16_t *y;
  uint16_t *shared_h;
  uint16_t *shared_out;
  int4 *work;
  int4 *tiles;         // grouped-GEMM row tiles {expert, first position, rows, 0}
  int32_t *chunk_counts;  // multi-workgroup dispatch: per-chunk expert counts, then bases
  int32_t *num_tiles;
  int max_tiles;
  void *x_split;   // grouped GEMMs: FP8 hi/lo split of x [T][d] and of h [P][I]
  void *h_split;
  float *gp, *up;  // decode shared-expert gate/up partials [skq][T][Is]
  float *yp;       // decode shared-expert down partials [skd][T][d]
  uint16_t *router_split;  // many tokens: the router weights split into three bf16 parts
  size_t bytes;
};

// Carves the workspace; with base == nullptr only computes the size.
Workspace carve(char *base, int T, int d, int E, int k, int I, int Is) {
  Workspace w{};
  size_t off = 0;
  const size_t P = (size_t)T * k;
  auto take = [&](size_t bytes) -> char * {
    char *p = base ? base + off : nullptr;
    off += align_up(bytes);
    return p;
  };
  w.logits = (float *)take((size_t)T * E * 4);
  w.weights = (float *)take(P * 4);
  w.indices = (uint32_t *)take(P * 4);
  w.counts = (int32_t *)take((size_t)E * 4);
  w.offsets = (int32_t *)take((size_t)(E + 1) * 4);
  w.active = (int32_t *)take((size_t)E * 4);
  w.num_active = (int32_t *)take(4);
  w.status = (int32_t *)take(4);
  w.perm = (int32_t *)take(P * 4);
  w.inv = (int32_t *)take(P * 4);
  w.pair_token = (int32_t *)take(P * 4);
  w.h = (uint16_t *)take(P * I * 2);
  w.y = (uint16_t *)take(P * d * 2);
  w.shared_h = (uint16_t *)take((size_t)T * (Is > 0 ? Is : 0) * 2);
  w.shared_out = (uint16_t *)take((size_t)T * (Is > 0 ? d : 0) * 2);
  w.work = (int4 *)take((size_t)E * sizeof(int4));
  w.max_tiles = (int)((P + glm_grouped_tile_rows() - 1) / glm_grouped_tile_rows()) + E;
  w.tiles = (int4 *)take((size_t)w.max_tiles * sizeof(int4));
  w.num_tiles = (int32_t *)take(4);
  w.chunk_counts = (int32_t *)take(glm_dispatch_chunk_ints((long long)P, E) * 4);
  if (d % 32 == 0 && I % 32 == 0) {
    w.x_split = take(glm_act_split_bytes((long long)T, d));
    w.h_split = take(glm_act_split_bytes((long long)P, I));
  }
  const size_t tis = (size_t)T * (Is > 0 ? Is : 0) * 4;
  const int skq = d % 512 == 0 ? d / 512 : 1;
  const int skd = Is >= 128 ? Is / 128 : 1;  // bound on the down K split
  w.gp = (float *)take(tis * skq);
  w.up = (float *)take(tis * skq);
  w.yp = (float *)take((size_t)T * (Is > 0 ? d : 0) * 4 * skd);
  w.router_split =
      (uint16_t *)take(glm_router_split_supported(T, d) ? glm_router_split_bytes(E, d) : 0);
  w.bytes = off;
  return w;
}

}  // namespace

// ---------------------------------------------------------------- static scratch

// The workspace of glm_moe_forward_noalloc: a file-scope device array, one
// copy per device that loads the library, held until the process ends.  On
// the host, `scratch` names a stand-in, not the device copy: host code only
// ever uses the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[GLM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device ordinal

// The device address of `scratch` on the current device, looked up once per
// device (with that device current).  The stream must belong to that device:
// its kernels would otherwise take another device's address.
int noalloc_scratch(hipStream_t stream, void **out) {
  int dev = -1;
  GLM_HIP_CHECK(hipGetDevice(&dev));
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    GLM_HIP_CHECK(hipStreamGetDevice(stream, &sdev));
    GLM_REQUIRE(sdev == dev, GLM_ERR_INVALID_ARGUMENT,
                "moe_forward_noalloc: the stream belongs to device %d but device %d is current",
                (int)sdev, dev);
  }
  GLM_REQUIRE(dev >= 0 && dev < kMaxDevices, GLM_ERR_INVALID_ARGUMENT,
              "moe_forward_noalloc: device ordinal %d is out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void *ptr = nullptr;
    GLM_HIP_CHECK(hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch)));
    GLM_REQUIRE(ptr != nullptr && (reinterpret_cast<uintptr_t>(ptr) & 255u) == 0, GLM_ERR_HIP,
                "moe_forward_noalloc: unusable scratch address on device %d", dev);
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GLM_OK;
}

}  // namespace

extern "C" size_t glm_moe_workspace_bytes(int T, int d, int E, int top_k, int I, int I_shared) {
  if (T < 0 || d <= 0 || E <= 0 || top_k <= 0 || I <= 0) return 0;
  return carve(nullptr, T, d, E, top_k, I, I_shared).bytes;
}

extern "C" int glm_moe_workspace_init(void *stream, void *workspace, size_t workspace_bytes) {
  glm::clear_error();
  GLM_REQUIRE(workspace != nullptr, GLM_ERR_INVALID_ARGUMENT, "workspace_init: null workspace");
  GLM_REQUIRE(glm_aligned16({workspace}) && workspace_bytes % 4 == 0, GLM_ERR_INVALID_ARGUMENT,
              "workspace_init: workspace must be 16-byte aligned and a multiple of 4 bytes");
  return glm_fill_zero_launch((hipStream_t)stream, workspace, workspace_bytes);
}

int glm_hc_post_launch(hipStream_t stream, const glm::HcFuse &f, const float *y, int T, int d);

static int moe_forward_core(void *stream_v, const uint16_t *x, int T, int d,
                            const float *router_weight, const float *router_bias, int E,
                            int top_k, int n_group, int topk_group, int norm_topk_prob,
                            float routed_scaling_factor, int I, const uint8_t *gate_packed,
                            const uint8_t *gate_scales, const uint8_t *up_packed,
                            const uint8_t *up_scales, const uint8_t *down_packed,
                            const uint8_t *down_scales, int I_shared, int shared_fmt,
                            const void *shared_gate, const uint8_t *shared_gate_scales,
                            const void *shared_up, const uint8_t *shared_up_scales,
                            const void *shared_down, const uint8_t *shared_down_scales,
                            const uint16_t *shared_in, float swiglu_limit, void *workspace,
                            size_t workspace_bytes, float *out, float *weights_out,
                            uint32_t *indices_out, const glm::HcFuse *hc, bool *hc_done,
                            bool noalloc, const uint8_t *sx_rows = nullptr,
                            long long sx_stride = 0);

extern "C" int glm_moe_forward(void *stream_v, const uint16_t *x, int T, int d,
                               const float *router_weight, const float *router_bias, int E,
                               int top_k, int n_group, int topk_group, int norm_topk_prob,
                               float routed_scaling_factor, int I, const uint8_t *gate_packed,
                               const uint8_t *gate_scales, const uint8_t *up_packed,
                               const uint8_t *up_scales, const uint8_t *down_packed,
                               const uint8_t *down_scales, int I_shared, int shared_fmt,
                               const void *shared_gate, const uint8_t *shared_gate_scales,
                               const void *shared_up, const uint8_t *shared_up_scales,
                               const void *shared_down, const uint8_t *shared_down_scales,
                               const uint16_t *shared_in, float swiglu_limit, void *workspace,
                               size_t workspace_bytes, float *out, float *weights_out,
                               uint32_t *indices_out) {
  glm::clear_error();
  bool done = false;
  return moe_forward_core(stream_v, x, T, d, router_weight, router_bias, E, top_k, n_group,
                          topk_group, norm_topk_prob, routed_scaling_factor, I, gate_packed,
                          gate_scales, up_packed, up_scales, down_packed, down_scales, I_shared,
                          shared_fmt, shared_gate, shared_gate_scales, shared_up,
                          shared_up_scales, shared_down, shared_down_scales, shared_in,
                          swiglu_limit, workspace, workspace_bytes, out, weights_out, indices_out,
                          nullptr, &done, false);
}

extern "C" int glm_moe_forward_noalloc(
    void *stream_v, const uint16_t *x, int T, int d, const float *router_weight,
    const float *router_bias, int E, int top_k, int n_group, int topk_group, int norm_topk_prob,
    float routed_scaling_factor, int I, const uint8_t *gate_packed, const uint8_t *gate_scales,
    const uint8_t *up_packed, const uint8_t *up_scales, const uint8_t *down_packed,
    const uint8_t *down_scales, int I_shared, int shared_fmt, const void *shared_gate,
    const uint8_t *shared_gate_scales, const void *shared_up, const uint8_t *shared_up_scales,
    const void *shared_down, const uint8_t *shared_down_scales, const uint16_t *shared_in,
    float swiglu_limit, float *out, float *weights_out, uint32_t *indices_out) {
  glm::clear_error();
  bool done = false;
  return moe_forward_core(stream_v, x, T, d, router_weight, router_bias, E, top_k, n_group,
                          topk_group, norm_topk_prob, routed_scaling_factor, I, gate_packed,
                          gate_scales, up_packed, up_scales, down_packed, down_scales, I_shared,
                          shared_fmt, shared_gate, shared_gate_scales, shared_up,
                          shared_up_scales, shared_down, shared_down_scales, shared_in,
                          swiglu_limit, nullptr, 0, out, weights_out, indices_out, nullptr, &done,
                          true);
}

extern "C" int glm_moe_forward_scalex(
    void *stream_v, const uint16_t *x, int T, int d, const float *router_weight,
    const float *router_bias, int E, int top_k, int n_group, int topk_group, int norm_topk_prob,
    float routed_scaling_factor, int I, const uint8_t *gate_packed, const uint8_t *up_packed,
    const uint8_t *down_packed, const uint8_t *scalex_rows, int64_t scalex_stride, int I_shared,
    int shared_fmt, const void *shared_gate, const uint8_t *shared_gate_scales,
    const void *shared_up, const uint8_t *shared_up_scales, const void *shared_down,
    const uint8_t *shared_down_scales, const uint16_t *shared_in, float swiglu_limit,
    void *workspace, size_t workspace_bytes, float *out, float *weights_out,
    uint32_t *indices_out) {
  glm::clear_error();
  GLM_REQUIRE(scalex_rows != nullptr, GLM_ERR_INVALID_ARGUMENT,
              "moe_forward_scalex: null scalex_rows");
  GLM_REQUIRE(scalex_stride > 0 && scalex_stride % 256 == 0 &&
                  ((uintptr_t)scalex_rows & 255u) == 0,
              GLM_ERR_INVALID_ARGUMENT,
              "moe_forward_scalex: the rows must be 256-byte aligned with a stride that is a "
              "positive multiple of 256 (stride %lld)",
              (long long)scalex_stride);
  GLM_REQUIRE(d % 128 == 0 && I % 128 == 0, GLM_ERR_UNSUPPORTED_SHAPE,
              "moe_forward_scalex: d=%d and I=%d must be multiples of 128", d, I);
  GLM_REQUIRE((long long)3 * I * (d / 32) < (1LL << 31), GLM_ERR_UNSUPPORTED_SHAPE,
              "moe_forward_scalex: %lld scales per expert exceed 2^31",
              (long long)3 * I * (d / 32));
  // the kernels read each row's directory and record header at fixed offsets
  const long long fixed = (long long)glm::scalex_dir_bytes((uint32_t)(3 * I * (d / 32))) + 24;
  GLM_REQUIRE(scalex_stride >= fixed, GLM_ERR_INVALID_ARGUMENT,
              "moe_forward_scalex: stride %lld is shorter than a row's directory and record "
              "header (%lld bytes)",
              (long long)scalex_stride, fixed);
  bool done = false;
  return moe_forward_core(stream_v, x, T, d, router_weight, router_bias, E, top_k, n_group,
                          topk_group, norm_topk_prob, routed_scaling_factor, I, gate_packed,
                          nullptr, up_packed, nullptr, down_packed, nullptr, I_shared, shared_fmt,
                          shared_gate, shared_gate_scales, shared_up, shared_up_scales,
                          shared_down, shared_down_scales, shared_in, swiglu_limit, workspace,
                          workspace_bytes, out, weights_out, indices_out, nullptr, &done, false,
                          scalex_rows, scalex_stride);
}

extern "C" int glm_moe_forward_hc(void *stream_v, const uint16_t *x, int T, int d,
                                  const float *router_weight, const float *router_bias, int E,
                                  int top_k, int n_group, int topk_group, int norm_topk_prob,
                                  float routed_scaling_factor, int I, const uint8_t *gate_packed,
                                  const uint8_t *gate_scales, const uint8_t *up_packed,
                                  const uint8_t *up_scales, const uint8_t *down_packed,
                                  const uint8_t *down_scales, int I_shared, int shared_fmt,
                                  const void *shared_gate, const uint8_t *shared_gate_scales,
                                  const void *shared_up, const uint8_t *shared_up_scales,
                                  const void *shared_down, const uint8_t *shared_down_scales,
                                  const uint16_t *shared_in, float swiglu_limit, void *workspace,
                                  size_t workspace_bytes, float *out, float *weights_out,
                                  uint32_t *indices_out, const float *residual, int hc,
                                  const float *post, const float *comb, int flags,
                                  float *hc_out) {
  glm::clear_error();
  GLM_REQUIRE(residual && post && comb && hc_out, GLM_ERR_INVALID_ARGUMENT,
              "moe_forward_hc: null hyper-connection argument");
  GLM_REQUIRE(hc >= 1 && hc <= 8, GLM_ERR_UNSUPPORTED_SHAPE, "moe_forward_hc: hc_mult %d > 8",
              hc);
  GLM_REQUIRE((flags & ~GLM_HC_BF16_STREAMS) == 0, GLM_ERR_INVALID_ARGUMENT,
              "moe_forward_hc: unknown flags %d", flags);
  GLM_REQUIRE(d % 4 == 0 && glm_aligned16({residual, hc_out}), GLM_ERR_INVALID_ARGUMENT,
              "moe_forward_hc: residual and hc_out must be 16-byte aligned, d %% 4 == 0");
  const glm::HcFuse f{residual, post, comb, hc_out, hc, (flags & GLM_HC_BF16_STREAMS) != 0};
  bool done = false;
  int rc = moe_forward_core(stream_v, x, T, d, router_weight, router_bias, E, top_k, n_group,
                            topk_group, norm_topk_prob, routed_scaling_factor, I, gate_packed,
                            gate_scales, up_packed, up_scales, down_packed, down_scales,
                            I_shared, shared_fmt, shared_gate, shared_gate_scales, shared_up,
                            shared_up_scales, shared_down, shared_down_scales, shared_in,
                            swiglu_limit, workspace, workspace_bytes, out, weights_out,
                            indices_out, &f, &done, false);
  if (rc != GLM_OK || done || T == 0) return rc;
  return glm_hc_post_launch((hipStream_t)stream_v, f, out, T, d);
}

static int moe_forward_core(void *stream_v, const uint16_t *x, int T, int d,
                            const float *router_weight, const float *router_bias, int E,
                            int top_k, int n_group, int topk_group, int norm_topk_prob,
                            float routed_scaling_factor, int I, const uint8_t *gate_packed,
                            const uint8_t *gate_scales, const uint8_t *up_packed,
                            const uint8_t *up_scales, const uint8_t *down_packed,
                            const uint8_t *down_scales, int I_shared, int shared_fmt,
                            const void *shared_gate, const uint8_t *shared_gate_scales,
                            const void *shared_up, const uint8_t *shared_up_scales,
                            const void *shared_down, const uint8_t *shared_down_scales,
                            const uint16_t *shared_in, float swiglu_limit, void *workspace,
                            size_t workspace_bytes, float *out, float *weights_out,
                            uint32_t *indices_out, const glm::HcFuse *hc, bool *hc_done,
                            bool noalloc, const uint8_t *sx_rows, long long sx_stride) {
  hipStream_t stream = (hipStream_t)stream_v;
  GLM_REQUIRE(x && router_weight && router_bias && gate_packed && up_packed && down_packed &&
                  (sx_rows || (gate_scales && up_scales && down_scales)) &&
                  (workspace || noalloc) && out,
              GLM_ERR_INVALID_ARGUMENT, "moe_forward: null pointer argument");
  GLM_REQUIRE(T >= 0 && d > 0 && E > 0 && top_k > 0 && I > 0, GLM_ERR_INVALID_ARGUMENT,
              "moe_forward: invalid sizes T=%d d=%d E=%d k=%d I=%d", T, d, E, top_k, I);
  GLM_REQUIRE((long long)T * top_k < (1LL << 30), GLM_ERR_UNSUPPORTED_SHAPE,
              "moe_forward: T*k = %lld pairs exceeds 2^30", (long long)T * top_k);
  GLM_REQUIRE(d % 32 == 0 && I % 32 == 0, GLM_ERR_UNSUPPORTED_SHAPE,
              "moe_forward: d=%d and I=%d must be multiples of 32", d, I);
  GLM_REQUIRE(E <= 448, GLM_ERR_UNSUPPORTED_SHAPE, "moe_forward: E=%d exceeds 448", E);
  const bool has_shared = shared_gate != nullptr;
  GLM_REQUIRE(!has_shared || (shared_up && shared_down && I_shared > 0 && I_shared % 32 == 0),
              GLM_ERR_INVALID_ARGUMENT, "moe_forward: incomplete shared expert (I_shared=%d)",
              I_shared);
  GLM_REQUIRE(shared_fmt == GLM_FMT_BF16 || shared_fmt == GLM_FMT_MXFP8 ||
                  shared_fmt == GLM_FMT_MXFP4,
              GLM_ERR_INVALID_ARGUMENT, "moe_forward: unknown shared format %d", shared_fmt);
  GLM_REQUIRE(!has_shared || shared_fmt == GLM_FMT_BF16 ||
                  (shared_gate_scales && shared_up_scales && shared_down_scales),
              GLM_ERR_INVALID_ARGUMENT, "moe_forward: MX shared expert needs scales");
  int rc = glm_router_validate(x, T, d, router_weight, router_bias, E, top_k, n_group,
                               topk_group, out, out);
  if (rc != GLM_OK) return rc;
  GLM_REQUIRE(glm_aligned16({x, router_weight, router_bias, gate_packed, up_packed, down_packed,
                              shared_gate, shared_up, shared_down, shared_in, workspace, out,
                              weights_out, indices_out}),
              GLM_ERR_INVALID_ARGUMENT, "moe_forward: buffers must be 16-byte aligned");
  const Workspace need = carve(nullptr, T, d, E, top_k, I, has_shared ? I_shared : 0);
  if (noalloc) {
    GLM_REQUIRE(need.bytes <= (size_t)GLM_NOALLOC_SCRATCH_BYTES, GLM_ERR_WORKSPACE,
                "moe_forward_noalloc: these sizes need %zu bytes of workspace, above the "
                "%zu-byte scratch array",
                need.bytes, (size_t)GLM_NOALLOC_SCRATCH_BYTES);
  } else {
    GLM_REQUIRE(workspace_bytes >= need.bytes, GLM_ERR_WORKSPACE,
                "moe_forward: workspace of %zu bytes is below the %zu required", workspace_bytes,
                need.bytes);
  }
  if (T == 0) return GLM_OK;
  if (noalloc) {
    rc = noalloc_scratch(stream, &workspace);
    if (rc != GLM_OK) return rc;
  }
  Workspace w = carve((char *)workspace, T, d, E, top_k, I, has_shared ? I_shared : 0);
  float *wts = weights_out ? weights_out : w.weights;
  uint32_t *idx = indices_out ? indices_out : w.indices;

  const int Is = has_shared ? I_shared : 0;
  const bool shared_bf16 = has_shared && shared_fmt == GLM_FMT_BF16;
  const uint16_t *shared_ready = shared_in;  // caller-computed shared output, if any
  const bool fuse_shared = shared_bf16 && !shared_in;
  GLM_REQUIRE(!sx_rows || glm_pair_path_supported(T, d, E, top_k, I, fuse_shared ? Is : 0),
              GLM_ERR_UNSUPPORTED_SHAPE,
              "moe_forward_scalex: coded scales are decoded by the few-token kernels, which take "
              "T <= 4, top_k <= 8, d / 512 in {2, 4, 6, 8} and I / 128 in {1, 2, 4, 6, 8, 16} "
              "(T=%d d=%d k=%d I=%d)",
              T, d, top_k, I);
  if (glm_pair_path_supported(T, d, E, top_k, I, fuse_shared ? Is : 0)) {
    // a few tokens: three token-major kernels, no dispatch
    if (has_shared && !shared_in && !shared_bf16) {
      rc = glm_mlp_launch(stream, x, T, d, I_shared, shared_fmt, shared_gate, shared_gate_scales,
                          shared_up, shared_up_scales, shared_down, shared_down_scales,
                          swiglu_limit, w.shared_h, w.shared_out);
      if (rc) return rc;
      shared_ready = w.shared_out;
    }
    rc = glm_pair_path_launch(
        stream, x, T, d, router_weight, router_bias, E, top_k, n_group, topk_group,
        norm_topk_prob, routed_scaling_factor, w.logits, wts, idx, I, gate_packed, gate_scales,
        up_packed, up_scales, down_packed, down_scales,
        fuse_shared ? (const uint16_t *)shared_gate : nullptr,
        fuse_shared ? (const uint16_t *)shared_up : nullptr,
        fuse_shared ? (const uint16_t *)shared_down : nullptr, Is, w.gp, w.up, w.shared_h, w.yp,
        shared_ready, w.h, swiglu_limit, out, hc, sx_rows, sx_stride);
    *hc_done = hc != nullptr;  // fused into the down + combine kernel
    return rc;
  }
  if (glm_decode_path_supported(T, d, E, top_k, I, fuse_shared ? Is : 0)) {
    // decode: six short kernels, no host synchronisation; the bf16 shared
    // expert rides in the two routing kernels, or from 16 tokens on (router
    // logits on MFMA) in the two routed expert kernels
    const bool in_experts = fuse_shared && glm_decode_shared_in_experts(T, d);
    const bool in_route = fuse_shared && !in_experts;
    const uint16_t *sg = (const uint16_t *)shared_gate, *su = (const uint16_t *)shared_up,
                   *sd = (const uint16_t *)shared_down;
    rc = glm_route_decode_launch(
        stream, x, T, d, router_weight, router_bias, E, top_k, n_group, topk_group,
        norm_topk_prob, routed_scaling_factor, w.logits, wts, idx, w.counts, w.offsets, w.perm,
        w.inv, w.pair_token, w.active, w.num_active, w.status, w.work, in_route ? sg : nullptr,
        in_route ? su : nullptr, in_route ? sd : nullptr, Is, w.gp, w.up, w.shared_h, w.yp,
        swiglu_limit);
    if (rc) return rc;
    rc = glm_decode_gate_up_launch(stream, x, T, d, I, E, top_k, gate_packed, gate_scales,
                                   up_packed, up_scales, w.pair_token, w.work, w.h, swiglu_limit,
                                   in_experts ? sg : nullptr, in_experts ? su : nullptr, Is,
                                   w.shared_h);
    if (rc) return rc;
    rc = glm_decode_down_launch(stream, w.h, T, top_k, I, d, E, down_packed, down_scales, w.work,
                                w.y, in_experts ? sd : nullptr, Is, w.shared_h, w.yp);
    if (rc) return rc;
    if (fuse_shared)
      return glm_combine_parts_launch(stream, w.y, w.inv, wts, nullptr, w.yp,
                                      glm_decode_shared_skd(Is), T, top_k, d, out);
    if (has_shared && !shared_in) {
      rc = glm_mlp_launch(stream, x, T, d, I_shared, shared_fmt, shared_gate, shared_gate_scales,
                          shared_up, shared_up_scales, shared_down, shared_down_scales,
                          swiglu_limit, w.shared_h, w.shared_out);
      if (rc) return rc;
      shared_ready = w.shared_out;
    }
    return glm_combine_launch(stream, w.y, w.inv, wts, shared_ready, T, top_k, d, out);
  }
  // general path: dispatch, then the grouped MFMA GEMMs over 128-row tiles
  // for more than 64 tokens when the shape allows, else the tiled GEMV
  // kernels over the work list (a few tokens in a 128-row tile would be
  // mostly padding)
  // (the grouped GEMMs address the FP8 splits of x and h with 32-bit offsets:
  // beyond 4 GiB of split the layer stays on the GEMV kernels)
  const bool grouped = glm_grouped_supported(d, I) && T > 64 && glm_split_fits(T, d) &&
                       glm_split_fits((long long)T * top_k, I);
  // with the bf16 router GEMM, x's FP8 split rides in the router weights'
  // split launch (one kernel, two block ranges)
  const bool split_early = grouped && w.router_split != nullptr && glm_router_split_supported(T, d);
  if (split_early) {
    rc = glm_prefill_split_launch(stream, router_weight, E, d, w.router_split, x, T, w.x_split);
    if (rc) return rc;
  }
  rc = glm_router_launch(stream, x, T, d, router_weight, router_bias, E, top_k, n_group,
                         topk_group, norm_topk_prob, routed_scaling_factor, w.logits, wts, idx,
                         w.router_split, split_early);
  if (rc) return rc;
  rc = glm_dispatch_launch(stream, idx, T, top_k, E, w.counts, w.offsets, w.perm, w.inv,
                           w.pair_token, w.active, w.num_active, w.work, w.status,
                           grouped ? glm_grouped_tile_rows() : 0, grouped ? w.tiles : nullptr,
                           grouped ? w.num_tiles : nullptr, w.chunk_counts);
  if (rc) return rc;
  bool shared_fused = false;
  if (grouped) {
    if (!split_early) {
      rc = glm_act_split_launch(stream, x, T, d, w.x_split);
      if (rc) return rc;
    }
    // a bf16 shared expert on the dense GEMMs: its gate/up tiles ride in the
    // routed gate/up launch (after the routed work items)
    shared_fused = has_shared && !shared_in &&
                   glm_grouped_dense_mlp_supported(T, d, I_shared, shared_fmt);
    if (shared_fused)
      rc = glm_grouped_gate_up_shared_launch(
          stream, w.x_split, T, w.pair_token, w.tiles, w.num_tiles, w.max_tiles, d, I,
          gate_packed, gate_scales, up_packed, up_scales, w.h, swiglu_limit, w.h_split,
          (long long)T * top_k, x, I_shared, static_cast<const uint16_t *>(shared_gate),
          static_cast<const uint16_t *>(shared_up), w.shared_h);
    else
      rc = glm_grouped_gate_up_launch(stream, w.x_split, T, w.pair_token, w.tiles, w.num_tiles,
                                      w.max_tiles, d, I, gate_packed, gate_scales, up_packed,
                                      up_scales, w.h, swiglu_limit, w.h_split, (long long)T * top_k);
    if (rc) return rc;  // the gate/up epilogue writes h's FP8 split for the down GEMM
    rc = glm_grouped_down_launch(stream, w.h_split, (long long)T * top_k, w.tiles, w.num_tiles,
                                 w.max_tiles, I, d, down_packed, down_scales, w.y);
  } else {
    rc = glm_gate_up_launch(stream, x, T, d, I, E, top_k, gate_packed, gate_scales, up_packed,
                            up_scales, w.pair_token, w.work, swiglu_limit, w.h);
    if (rc) return rc;
    rc = glm_down_launch(stream, w.h, T, top_k, I, d, E, down_packed, down_scales, w.work, w.y);
  }
  if (rc) return rc;
  if (has_shared && !shared_in) {
    if (shared_fused)
      rc = glm_grouped_dense_down_launch(stream, w.shared_h, T, I_shared, d,
                                         static_cast<const uint16_t *>(shared_down), w.shared_out);
    else
      rc = glm_mlp_launch(stream, x, T, d, I_shared, shared_fmt, shared_gate, shared_gate_scales,
                          shared_up, shared_up_scales, shared_down, shared_down_scales,
                          swiglu_limit, w.shared_h, w.shared_out);
    if (rc) return rc;
    shared_ready = w.shared_out;
  }
  return glm_combine_launch(stream, w.y, w.inv, wts, shared_ready, T, top_k, d, out);
}
