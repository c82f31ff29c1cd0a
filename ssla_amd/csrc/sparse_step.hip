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

namespace ssla {
namespace {

template <int K, int V>
__global__ __launch_bounds__(256) void sparse_gla_step_kernel(
    const int32_t *__restrict__ site_idx, int n_active, const float *__restrict__ q,
    const float *__restrict__ k, const float *__restrict__ v, const float *__restrict__ g,
    float *__restrict__ state, int n_sites, int H, float scale, float *__restrict__ o,
    int32_t *__restrict__ status) {
  constexpr int VL = V / 4;          // lanes per state row (float4 each)
  constexpr int RG = 64 / VL;        // row groups per wavefront
  constexpr int RPL = K / RG;        // rows per lane
  static_assert(RPL >= 1 && RG * RPL == K, "unsupported K/V");
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= static_cast<int64_t>(n_active) * H) return;
  const int i = static_cast<int>(item / H);
  const int h = static_cast<int>(item % H);
  const int site = site_idx[i];
  const int vc = lane % VL;          // float4 column
  const int rg = lane / VL;          // row group: rows rg*RPL .. rg*RPL+RPL-1
  const int64_t io = static_cast<int64_t>(i) * H + h;
  if (site < 0 || site >= n_sites || (i > 0 && site_idx[i - 1] >= site)) {
    if (rg == 0) reinterpret_cast<float4 *>(o + io * V)[vc] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (status && lane == 0) __hip_atomic_store(status, SSLA_ERR_ARG, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const float4 vv = reinterpret_cast<const float4 *>(v + io * V)[vc];
  float4 *S = reinterpret_cast<float4 *>(state + (static_cast<int64_t>(site) * H + h) * K * V);

  float4 s[RPL];
#pragma unroll
  for (int r = 0; r < RPL; ++r) s[r] = S[(rg * RPL + r) * VL + vc];

  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int row = rg * RPL + r;
    const float gg = g[io * K + row];
    const float kk = k[io * K + row];
    const float qq = q[io * K + row] * scale;
    const float d = fast_exp2(gg * kLog2e);
    s[r].x = fmaf(d, s[r].x, kk * vv.x);
    s[r].y = fmaf(d, s[r].y, kk * vv.y);
    s[r].z = fmaf(d, s[r].z, kk * vv.z);
    s[r].w = fmaf(d, s[r].w, kk * vv.w);
    acc.x = fmaf(qq, s[r].x, acc.x);
    acc.y = fmaf(qq, s[r].y, acc.y);
    acc.z = fmaf(qq, s[r].z, acc.z);
    acc.w = fmaf(qq, s[r].w, acc.w);
  }
#pragma unroll
  for (int r = 0; r < RPL; ++r) S[(rg * RPL + r) * VL + vc] = s[r];

#pragma unroll
  for (int m = VL; m < 64; m <<= 1) {
    acc.x += __shfl_xor(acc.x, m);
    acc.y += __shfl_xor(acc.y, m);
    acc.z += __shfl_xor(acc.z, m);
    acc.w += __shfl_xor(acc.w, m);
  }
  if (rg == 0) reinterpret_cast<float4 *>(o + io * V)[vc] = acc;
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
  const int64_t blocks = (items + 3) / 4;
  SSLA_CHECK_ARG(blocks <= 0x7fffffff, "sparse_gla_step: too many active sites");
  dim3 grid(static_cast<unsigned>(blocks)), block(256);
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
