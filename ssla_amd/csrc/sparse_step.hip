// One time bin of the per-site matrix-state GLA update at active sites only.
//
//   S[site] <- diag(exp(g_i)) S[site] + k_i v_i^T,   o_i = (scale q_i)^T S[site]
//
// This is naive_gla_recurrent (reference ops/gla/naive.py:50-111) on a
// length-1 sequence whose initial state is the stored state of the site.
//
// One wavefront owns one (active site, head): the [K, V] fp32 state tile is
// read with 16-byte loads (a row of V floats is V/4 lanes), updated in
// registers and written back; o needs a reduction over the key rows held by
// the other lane groups.  Only rows named by site_idx are touched, so the
// states of inactive sites stay bit-identical.  The kernel is a pure HBM
// stream: 2*K*V*4 bytes of state plus (3K + 2V)*4 bytes of q/k/g/v/o per
// (site, head).
//
// The site list must be strictly increasing and inside [0, n_sites): an
// entry that is not (out of range, or not above the entry before it -- a
// duplicate or an unsorted list) is skipped: its o rows are written as
// zeros, no state is touched, and the status word (if given) is set to
// SSLA_ERR_ARG.  A strictly increasing list also rules out two wavefronts
// updating one state tile.
#include "common.h"

#ifndef SSLA_SS_IPW
#define SSLA_SS_IPW 1
#endif
#ifndef SSLA_SS_WPB
#define SSLA_SS_WPB 1
#endif

namespace ssla {
namespace {

constexpr int kStepWaves = SSLA_SS_WPB;   // wavefronts per workgroup
constexpr int kStepItems = SSLA_SS_IPW;   // (site, head) items per wavefront

// Sum over the lanes l, l ^ VL, l ^ 2 VL, ... (the row groups that hold one
// float4 column): rotations inside each 16-lane DPP row (by 8, then by 4:
// a sum is the same under either pairing), then v_permlane16_swap /
// v_permlane32_swap across rows -- VALU lane moves, no LDS round trips.
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, x), 0x120 + N, 0xf, 0xf, false));
}
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
template <int VL>
__device__ __forceinline__ float sum_row_groups(float x) {
  if constexpr (VL <= 8) x += row_ror<8>(x);
  if constexpr (VL <= 4) x += row_ror<4>(x);
  const u32x2 a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a.x) + __uint_as_float(a.y);
  const u32x2 b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b.x) + __uint_as_float(b.y);
}

template <int K, int V>
__global__ __launch_bounds__(64 * kStepWaves) void sparse_gla_step_kernel(
    const int32_t *__restrict__ site_idx, int n_active, const float *__restrict__ q,
    const float *__restrict__ k, const float *__restrict__ v, const float *__restrict__ g,
    float *__restrict__ state, int n_sites, int H, float scale, float *__restrict__ o,
    int32_t *__restrict__ status) {
  constexpr int VL = V / 4;          // lanes per state row (float4 each)
  constexpr int RG = 64 / VL;        // row groups per wavefront
  constexpr int RPL = K / RG;        // rows per lane
  static_assert(RPL >= 1 && RG * RPL == K && VL >= 4 && VL <= 16, "unsupported K/V");
  const int lane = threadIdx.x & 63;
  // wavefront-uniform: the (site, head) indexing runs on the scalar unit
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n_items = n_active * H;   // < 2^31 (host check)
  const int item0 = (static_cast<int>(blockIdx.x) * kStepWaves + wv) * kStepItems;
  if (item0 >= n_items) return;
  const int vc = lane % VL;          // float4 column
  const int rg = lane / VL;          // row group: rows rg*RPL .. rg*RPL+RPL-1
  // every item's inputs first (they do not depend on the site index, so
  // their loads overlap its load), then every item's state, then the math
  float4 vv[kStepItems];
  float gg[kStepItems][RPL], kk[kStepItems][RPL], qq[kStepItems][RPL];
  int site[kStepItems];
#pragma unroll
  for (int u = 0; u < kStepItems; ++u) {
    const int item = min(item0 + u, n_items - 1);
    const int64_t io = static_cast<int64_t>(item / H) * H + item % H;
    vv[u] = reinterpret_cast<const float4 *>(v + io * V)[vc];
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      const int row = rg * RPL + r;
      gg[u][r] = g[io * K + row];
      kk[u][r] = k[io * K + row];
      qq[u][r] = q[io * K + row];
    }
    site[u] = site_idx[item / H];
  }
  float4 s[kStepItems][RPL];
  bool ok[kStepItems];
#pragma unroll
  for (int u = 0; u < kStepItems; ++u) {
    const int item = min(item0 + u, n_items - 1);
    const int i = item / H, h = item % H;
    ok[u] = item0 + u < n_items && site[u] >= 0 && site[u] < n_sites && !(i > 0 && site_idx[i - 1] >= site[u]);
    if (ok[u]) {
      const float4 *S = reinterpret_cast<const float4 *>(state + (static_cast<int64_t>(site[u]) * H + h) * K * V);
#pragma unroll
      for (int r = 0; r < RPL; ++r) s[u][r] = S[(rg * RPL + r) * VL + vc];
    }
  }
#pragma unroll
  for (int u = 0; u < kStepItems; ++u) {
    if (item0 + u >= n_items) break;   // wavefront-uniform
    const int item = item0 + u;
    const int h = item % H;
    const int64_t io = static_cast<int64_t>(item / H) * H + h;
    if (!ok[u]) {
      if (rg == 0) reinterpret_cast<float4 *>(o + io * V)[vc] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (status && lane == 0) __hip_atomic_store(status, SSLA_ERR_ARG, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }
    float4 *S = reinterpret_cast<float4 *>(state + (static_cast<int64_t>(site[u]) * H + h) * K * V);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      const float d = fast_exp2(gg[u][r] * kLog2e);
      const float qs = qq[u][r] * scale;
      s[u][r].x = fmaf(d, s[u][r].x, kk[u][r] * vv[u].x);
      s[u][r].y = fmaf(d, s[u][r].y, kk[u][r] * vv[u].y);
      s[u][r].z = fmaf(d, s[u][r].z, kk[u][r] * vv[u].z);
      s[u][r].w = fmaf(d, s[u][r].w, kk[u][r] * vv[u].w);
      acc.x = fmaf(qs, s[u][r].x, acc.x);
      acc.y = fmaf(qs, s[u][r].y, acc.y);
      acc.z = fmaf(qs, s[u][r].z, acc.z);
      acc.w = fmaf(qs, s[u][r].w, acc.w);
    }
#pragma unroll
    for (int r = 0; r < RPL; ++r) S[(rg * RPL + r) * VL + vc] = s[u][r];
    acc.x = sum_row_groups<VL>(acc.x);
    acc.y = sum_row_groups<VL>(acc.y);
    acc.z = sum_row_groups<VL>(acc.z);
    acc.w = sum_row_groups<VL>(acc.w);
    if (rg == 0) reinterpret_cast<float4 *>(o + io * V)[vc] = acc;
  }
}

}  // namespace
}  // namespace ssla

extern "C" int ssla_sparse_gla_step(const int32_t *site_idx, int n_active, const float *q,
                                    const float *k, const float *v, const float *g,
                                    float *state, int n_sites, int H, int K, int V, float scale,
                                    float *o, int32_t *status, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_active >= 0 && n_sites >= 0 && H > 0,
                 "sparse_gla_step: bad sizes n_active=%d n_sites=%d H=%d", n_active, n_sites, H);
  if (n_active == 0) return SSLA_OK;
  SSLA_CHECK_ARG(site_idx && q && k && v && g && state && o, "sparse_gla_step: null pointer");
  SSLA_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(g, 16) &&
                     aligned(state, 16) && aligned(o, 16),
                 "sparse_gla_step: tensors must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t items = static_cast<int64_t>(n_active) * H;
  const int64_t blocks = (items + kStepWaves * kStepItems - 1) / (kStepWaves * kStepItems);
  SSLA_CHECK_ARG(items <= 0x7fffffff, "sparse_gla_step: too many active sites");
  dim3 grid(static_cast<unsigned>(blocks)), block(64 * kStepWaves);
#define SSLA_STEP(KK, VV)                                                                       \
  if (K == KK && V == VV) {                                                                     \
    hipLaunchKernelGGL((sparse_gla_step_kernel<KK, VV>), grid, block, 0, st, site_idx, n_active, \
                       q, k, v, g, state, n_sites, H, scale, o, status);                        \
    return launch_status("sparse_gla_step");                                                    \
  }
  SSLA_STEP(16, 16) SSLA_STEP(16, 32) SSLA_STEP(16, 64)
  SSLA_STEP(32, 16) SSLA_STEP(32, 32) SSLA_STEP(32, 64)
  SSLA_STEP(64, 16) SSLA_STEP(64, 32) SSLA_STEP(64, 64)
#undef SSLA_STEP
  set_error("sparse_gla_step: K=%d V=%d not in {16,32,64}", K, V);
  return SSLA_ERR_UNSUPPORTED;
}
