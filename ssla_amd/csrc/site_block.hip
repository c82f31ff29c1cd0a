// Fused projections of the per-site GLA block of the asynchronous step
// (ssla_amd.backbone.SiteGLABlock), on bf16 matrix cores.
//
// ssla_site_project: q, k, v = bf16(x W^T) for W = Wq, Wk, Wv and the log
// gates g = logsigmoid(bf16(x Wg^T)) / gate_normalizer (fp32), from fp32
// event features x: the bf16 rounding of x, the four GEMMs and the gate
// nonlinearity in one launch.
// ssla_site_finish: y = LayerNorm(bf16(o Wo^T) + r) with r = bf16(x Wr^T)
// (an input projection) or x, in one launch.
// The rounding points are those of torch's bf16 F.linear (fp32 accumulation,
// one rounding of the result to bf16), so the results equal the module's
// composition of library calls up to the order of the fp32 sums.
//
// Layout: a workgroup of 4 wavefronts takes 64 event rows; wavefront w owns
// rows 16 w .. 16 w + 15 and every output column of its launch, as
// v_mfma_f32_16x16x32_bf16 tiles.  Operands come straight from global
// memory in the MFMA layout (lane l: row / column l % 16, reduction
// elements 8 (l / 16) .. + 7, one 16-byte piece), no LDS and no barriers;
// the weights are small and shared by every workgroup (cache resident).
// finish keeps a row's whole output in its wavefront, so LayerNorm reduces
// over the 16 lanes of a lane group (xor shuffles) with no LDS either.
#include "common.h"

namespace ssla {
namespace {

constexpr int kWaves = 4;
constexpr int kRows = 16 * kWaves;   // event rows per workgroup

typedef float f32x8v __attribute__((ext_vector_type(8)));

// Eight consecutive fp32 inputs of a row, rounded to bf16 (zeros when the
// row does not exist).
__device__ __forceinline__ bf16x8 a_from_f32(const float *x, int64_t row, int ld, int k, bool ok) {
  if (!ok) return bf16x8{};
  const float4 u = *reinterpret_cast<const float4 *>(x + row * ld + k);
  const float4 w = *reinterpret_cast<const float4 *>(x + row * ld + k + 4);
  const f32x8v v = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
  return __builtin_convertvector(v, bf16x8);
}

// Eight consecutive bf16 values of a row of a [rows, ld] bf16 matrix.
__device__ __forceinline__ bf16x8 bf16_piece(const uint16_t *p, int64_t row, int ld, int k, bool ok) {
  if (!ok) return bf16x8{};
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(p + row * ld + k));
}

__device__ __forceinline__ float round_bf16(float x) {
  return static_cast<float>(static_cast<__bf16>(x));
}

// grid (row tiles, 4 outputs q / k / v / g, column chunks of 128); w is
// [4 hd, cin] (the rows of Wq, Wk, Wv, Wg in turn).
__global__ __launch_bounds__(64 * kWaves) void site_project_kernel(const float *__restrict__ x, int64_t n, int cin,
                                                                   const uint16_t *__restrict__ w, int hd,
                                                                   float inv_gn, uint16_t *__restrict__ q,
                                                                   uint16_t *__restrict__ k, uint16_t *__restrict__ v,
                                                                   float *__restrict__ g) {
  constexpr int NT = 8;   // 128 columns
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 15, kq = 8 * (lane >> 4);
  const int which = blockIdx.y;
  const int c0 = blockIdx.z * 16 * NT;
  const int ncol = min(16 * NT, hd - c0);
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kRows + 16 * wv;
  const int64_t row = e0 + r;
  const bool rok = row < n;
  const uint16_t *wb = w + (static_cast<int64_t>(which) * hd + c0) * cin;
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < cin; k0 += 32) {
    const bf16x8 a = a_from_f32(x, row, cin, k0 + kq, rok);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (16 * t < ncol)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bf16_piece(wb, 16 * t + r, cin, k0 + kq, true), acc[t], 0,
                                                        0, 0);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (16 * t >= ncol) continue;
    const int col = c0 + 16 * t + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t ev = e0 + 4 * (lane >> 4) + i;
      if (ev >= n) continue;
      const float val = round_bf16(acc[t][i]);
      const int64_t o = ev * hd + col;
      if (which == 3) {
        g[o] = (fminf(val, 0.f) - log1pf(expf(-fabsf(val)))) * inv_gn;   // logsigmoid
      } else {
        uint16_t *dst = which == 0 ? q : which == 1 ? k : v;
        dst[o] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(val));
      }
    }
  }
}

// One wavefront: 16 rows x 16 NT output columns, LayerNorm over them.
template <int NT>
__global__ __launch_bounds__(64 * kWaves) void site_finish_kernel(const uint16_t *__restrict__ o, int64_t n, int hd,
                                                                  const uint16_t *__restrict__ wo,
                                                                  const float *__restrict__ x, int cin,
                                                                  const uint16_t *__restrict__ wr,
                                                                  const float *__restrict__ ln_w,
                                                                  const float *__restrict__ ln_b, float eps,
                                                                  float *__restrict__ y) {
  constexpr int C = 16 * NT;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 15, kq = 8 * (lane >> 4);
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kRows + 16 * wv;
  if (e0 >= n) return;   // whole wavefront (no barriers in this kernel)
  const int64_t row = e0 + r;
  const bool rok = row < n;
  f32x4 acc[NT], res[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = res[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < hd; k0 += 32) {
    const bf16x8 a = bf16_piece(o, row, hd, k0 + kq, rok);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bf16_piece(wo, 16 * t + r, hd, k0 + kq, true), acc[t], 0, 0,
                                                      0);
  }
  if (wr) {
    for (int k0 = 0; k0 < cin; k0 += 32) {
      const bf16x8 a = a_from_f32(x, row, cin, k0 + kq, rok);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        res[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bf16_piece(wr, 16 * t + r, cin, k0 + kq, true), res[t], 0,
                                                        0, 0);
    }
  }
  // y = bf16(o Wo^T) + (bf16(x Wr^T) or x); rows 4 (l / 16) + i of this
  // wavefront, columns 16 t + l % 16
  float yv[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t ev = e0 + 4 * (lane >> 4) + i;
      const float rv = wr ? round_bf16(res[t][i]) : (ev < n ? x[ev * cin + 16 * t + r] : 0.f);
      yv[t][i] = round_bf16(acc[t][i]) + rv;
    }
  // LayerNorm: the mean, then the mean squared deviation, each summed over
  // the NT tiles in the lane and over the 16 lanes of the lane group
  float mean[4], rstd[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) s += yv[t][i];
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) s += __shfl_xor(s, m);
    mean[i] = s / static_cast<float>(C);
    float d = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) d += (yv[t][i] - mean[i]) * (yv[t][i] - mean[i]);
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) d += __shfl_xor(d, m);
    rstd[i] = 1.f / sqrtf(d / static_cast<float>(C) + eps);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int col = 16 * t + r;
    const float lw = ln_w[col], lb = ln_b[col];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t ev = e0 + 4 * (lane >> 4) + i;
      if (ev < n) y[ev * C + col] = (yv[t][i] - mean[i]) * rstd[i] * lw + lb;
    }
  }
}

unsigned row_tiles(int64_t n) { return static_cast<unsigned>((n + kRows - 1) / kRows); }

}  // namespace
}  // namespace ssla

extern "C" int ssla_site_project(const float *x, int64_t n, int cin, const uint16_t *w, int hd, float gate_normalizer,
                                 uint16_t *q, uint16_t *k, uint16_t *v, float *g, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n >= 0 && cin > 0 && hd > 0 && gate_normalizer != 0.f,
                 "site_project: bad sizes n=%lld cin=%d hd=%d", (long long)n, cin, hd);
  if (cin % 32 != 0 || hd % 16 != 0) {
    set_error("site_project: needs cin a multiple of 32 and hd a multiple of 16 (cin=%d hd=%d)", cin, hd);
    return SSLA_ERR_UNSUPPORTED;
  }
  SSLA_CHECK_ARG(n < (int64_t{1} << 31) * kRows, "site_project: too many rows");
  if (n == 0) return SSLA_OK;
  SSLA_CHECK_ARG(x && w && q && k && v && g, "site_project: null pointer");
  SSLA_CHECK_ARG(aligned(x, 16) && aligned(w, 16), "site_project: x and w must be 16-byte aligned");
  hipLaunchKernelGGL(site_project_kernel, dim3(row_tiles(n), 4, (hd + 127) / 128), dim3(64 * kWaves), 0,
                     static_cast<hipStream_t>(stream), x, n, cin, w, hd, 1.f / gate_normalizer, q, k, v, g);
  return launch_status("site_project");
}

extern "C" int ssla_site_finish(const uint16_t *o, int64_t n, int hd, const uint16_t *wo, const float *x, int cin,
                                const uint16_t *wr, const float *ln_w, const float *ln_b, float eps, int cout,
                                float *y, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n >= 0 && hd > 0 && cin > 0 && cout > 0, "site_finish: bad sizes n=%lld hd=%d cin=%d cout=%d",
                 (long long)n, hd, cin, cout);
  if (hd % 32 != 0 || cin % 32 != 0 || !(cout == 16 || cout == 32 || cout == 64 || cout == 96 || cout == 128 ||
                                         cout == 192 || cout == 256)) {
    set_error("site_finish: needs hd, cin multiples of 32 and cout in {16, 32, 64, 96, 128, 192, 256} "
              "(hd=%d cin=%d cout=%d)", hd, cin, cout);
    return SSLA_ERR_UNSUPPORTED;
  }
  if (!wr && cin != cout) {
    set_error("site_finish: input size %d differs from output %d but no input projection given", cin, cout);
    return SSLA_ERR_ARG;
  }
  SSLA_CHECK_ARG(n < (int64_t{1} << 31) * kRows, "site_finish: too many rows");
  if (n == 0) return SSLA_OK;
  SSLA_CHECK_ARG(o && wo && x && ln_w && ln_b && y, "site_finish: null pointer");
  SSLA_CHECK_ARG(aligned(o, 16) && aligned(wo, 16) && aligned(x, 16) && (!wr || aligned(wr, 16)),
                 "site_finish: o, x and the weights must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
#define SITE_FINISH(NTV)                                                                                           \
  if (cout == 16 * NTV) {                                                                                          \
    hipLaunchKernelGGL((site_finish_kernel<NTV>), dim3(row_tiles(n)), dim3(64 * kWaves), 0, st, o, n, hd, wo, x,   \
                       cin, wr, ln_w, ln_b, eps, y);                                                                 \
    return launch_status("site_finish");                                                                           \
  }
  SITE_FINISH(1) SITE_FINISH(2) SITE_FINISH(4) SITE_FINISH(6) SITE_FINISH(8) SITE_FINISH(12) SITE_FINISH(16)
#undef SITE_FINISH
  return SSLA_ERR_UNSUPPORTED;
}
