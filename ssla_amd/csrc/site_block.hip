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
// over the 16 lanes of a lane group (xor shuffles) with no LDS either; at
// the step's four stage shapes it runs with both weight matrices resident
// in LDS (site_finish_resident_kernel: staged once per workgroup, no
// barrier per reduction step, the same sums in the same order).
#include "common.h"

namespace ssla {
namespace {

constexpr int kWaves = 4;
constexpr int kRows = 16 * kWaves;   // event rows per workgroup

typedef float f32x8v __attribute__((ext_vector_type(8)));

// Eight consecutive bf16 values of a row of a [rows, ld] bf16 matrix.
__device__ __forceinline__ bf16x8 bf16_piece(const uint16_t *p, int64_t row, int ld, int k, bool ok) {
  if (!ok) return bf16x8{};
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(p + row * ld + k));
}

__device__ __forceinline__ float round_bf16(float x) {
  return static_cast<float>(static_cast<__bf16>(x));
}

// grid (row tiles of 64 events, column chunks of 16 NTO); w is [4 hd, cin]
// (the rows of Wq, Wk, Wv, Wg in turn).  Wavefront w computes output w
// (q, k, v, g) for all 64 rows of the tile: 4 x NTO MFMA tiles, each weight
// piece reused by the 4 row tiles.  The tile's inputs are staged in LDS one
// 32-wide reduction step at a time as bf16 (shared by the 4 wavefronts),
// the next step's inputs loaded while the current step is multiplied (rows
// past n read row n - 1; their outputs are never stored); the results
// leave through a wave-private LDS block in 16-byte row pieces.
template <int NTO>
__global__ __launch_bounds__(64 * kWaves) void site_project_kernel(const float *__restrict__ x, int64_t n, int cin,
                                                                   const uint16_t *__restrict__ w, int hd,
                                                                   float inv_gn, uint16_t *__restrict__ q,
                                                                   uint16_t *__restrict__ k, uint16_t *__restrict__ v,
                                                                   float *__restrict__ g) {
  constexpr int NC = 16 * NTO;                          // columns of this launch's chunk
  __shared__ __align__(16) uint16_t xs[kRows][32 + 8];  // the tile's inputs, one k-step (bf16)
  __shared__ __align__(16) float ost[kWaves][16][NC + 4];   // one row tile of a wavefront's output
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r = lane & 15, kq = 8 * (lane >> 4);
  const int which = wv;
  const int c0 = blockIdx.y * NC;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kRows;
  const uint16_t *wb = w + (static_cast<int64_t>(which) * hd + c0) * cin;
  f32x4 acc[4][NTO];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < NTO; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // staging: thread -> (row tid / 4, inputs 8 (tid % 4) .. + 7)
  const int sr = tid >> 2, sk = 8 * (tid & 3);
  const int64_t srow = min(e0 + sr, n - 1);   // n > 0 (the launcher returns before)
  const float *xrow = x + srow * cin + sk;
  float4 xa = *reinterpret_cast<const float4 *>(xrow), xb = *reinterpret_cast<const float4 *>(xrow + 4);
  // the weight pieces of a step are loaded with the step before's inputs
  bf16x8 bn[NTO];
#pragma unroll
  for (int t = 0; t < NTO; ++t) bn[t] = bf16_piece(wb, 16 * t + r, cin, kq, true);
  for (int k0 = 0; k0 < cin; k0 += 32) {
    const f32x8v xf = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    bf16x8 bv[NTO];
#pragma unroll
    for (int t = 0; t < NTO; ++t) bv[t] = bn[t];
    if (k0 + 32 < cin) {
      xa = *reinterpret_cast<const float4 *>(xrow + k0 + 32);
      xb = *reinterpret_cast<const float4 *>(xrow + k0 + 36);
#pragma unroll
      for (int t = 0; t < NTO; ++t) bn[t] = bf16_piece(wb, 16 * t + r, cin, k0 + 32 + kq, true);
    }
    const bf16x8 xv = __builtin_convertvector(xf, bf16x8);
    __syncthreads();   // the previous step's reads of xs are done
    *reinterpret_cast<bf16x8 *>(&xs[sr][sk]) = xv;
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const bf16x8 av = *reinterpret_cast<const bf16x8 *>(&xs[16 * rt + r][kq]);
#pragma unroll
      for (int t = 0; t < NTO; ++t) acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv[t], acc[rt][t], 0, 0, 0);
    }
  }
  // results: row tile by row tile through this wavefront's LDS block
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
#pragma unroll
    for (int t = 0; t < NTO; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float val = round_bf16(acc[rt][t][i]);
        float outv = val;
        if (which == 3) {   // logsigmoid(val) / gate_normalizer
          const float e = __builtin_amdgcn_exp2f(-fabsf(val) * kLog2e);
          outv = (fminf(val, 0.f) - __builtin_amdgcn_logf(1.f + e) * 0.69314718055994531f) * inv_gn;
        }
        ost[wv][4 * (lane >> 4) + i][16 * t + r] = outv;
      }
    __syncthreads();
    const int64_t rbase = e0 + 16 * rt;
    if (which < 3) {
      // 16 rows x NC bf16: pieces of 8 values
      uint16_t *dst = which == 0 ? q : which == 1 ? k : v;
      constexpr int PR = NC / 8;   // pieces per row
      for (int p = lane; p < 16 * PR; p += 64) {
        const int rr = p / PR, cc = 8 * (p % PR);
        if (rbase + rr < n) {
          const float4 u = *reinterpret_cast<const float4 *>(&ost[wv][rr][cc]);
          const float4 u2 = *reinterpret_cast<const float4 *>(&ost[wv][rr][cc + 4]);
          const f32x8v f = {u.x, u.y, u.z, u.w, u2.x, u2.y, u2.z, u2.w};
          *reinterpret_cast<bf16x8 *>(dst + (rbase + rr) * hd + c0 + cc) = __builtin_convertvector(f, bf16x8);
        }
      }
    } else {
      constexpr int PR = NC / 4;
      for (int p = lane; p < 16 * PR; p += 64) {
        const int rr = p / PR, cc = 4 * (p % PR);
        if (rbase + rr < n)
          *reinterpret_cast<float4 *>(g + (rbase + rr) * hd + c0 + cc) =
              *reinterpret_cast<const float4 *>(&ost[wv][rr][cc]);
      }
    }
    __syncthreads();   // the block is rewritten by the next row tile
  }
}

// One wavefront: 16 rows x 16 NT output columns, LayerNorm over them.  The
// weights of each 32-wide reduction step are staged in LDS once per
// workgroup (shared by its 4 wavefronts); the next step's weight pieces and
// the next step's row pieces (o, then x) are loaded while the current step
// is multiplied, so the steps do not each wait on a memory round trip.
// Rows past n read row n - 1 (their results are never stored, and the
// LayerNorm sums stay within a row).
template <int NT>
__global__ __launch_bounds__(64 * kWaves) void site_finish_kernel(const uint16_t *__restrict__ o, int64_t n, int hd,
                                                                  const uint16_t *__restrict__ wo,
                                                                  const float *__restrict__ x, int cin,
                                                                  const uint16_t *__restrict__ wr,
                                                                  const float *__restrict__ ln_w,
                                                                  const float *__restrict__ ln_b, float eps,
                                                                  float *__restrict__ y) {
  constexpr int C = 16 * NT;
  constexpr int PT = (C * 4 + 64 * kWaves - 1) / (64 * kWaves);   // weight pieces per thread and step
  __shared__ __align__(16) uint16_t wst[C][32 + 8];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r = lane & 15, kq = 8 * (lane >> 4);
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kRows + 16 * wv;
  const int64_t row = min(e0 + r, n - 1);   // n > 0 (the launcher returns before)
  f32x4 acc[NT], res[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = res[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // o Wo^T (hd / 32 steps), then x Wr^T (cin / 32 steps) with an input
  // projection; each step's weights staged in LDS
  auto fetch = [&](const uint16_t *wm, int ld, int k0, uint4 (&pc)[PT]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int pc_i = tid + 64 * kWaves * j;   // piece: row pc_i / 4, inputs 8 (pc_i % 4) .. + 7
      pc[j] = pc_i < 4 * C ? *reinterpret_cast<const uint4 *>(wm + static_cast<int64_t>(pc_i >> 2) * ld + k0 +
                                                              8 * (pc_i & 3))
                           : uint4{0, 0, 0, 0};
    }
  };
  auto stage = [&](const uint4 (&pc)[PT]) __attribute__((always_inline)) {
    __syncthreads();   // the previous step's reads of wst are done
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int pc_i = tid + 64 * kWaves * j;
      if (pc_i < 4 * C) *reinterpret_cast<uint4 *>(&wst[pc_i >> 2][8 * (pc_i & 3)]) = pc[j];
    }
    __syncthreads();
  };
  // this lane's row pieces: o as bf16, x as fp32 (rounded when used)
  auto o_piece = [&](int k0) __attribute__((always_inline)) {
    return *reinterpret_cast<const uint4 *>(o + row * hd + k0 + kq);
  };
  auto x_piece = [&](int k0, float4 (&xv)[2]) __attribute__((always_inline)) {
    xv[0] = *reinterpret_cast<const float4 *>(x + row * cin + k0 + kq);
    xv[1] = *reinterpret_cast<const float4 *>(x + row * cin + k0 + kq + 4);
  };
  uint4 pcur[PT];
  fetch(wo, hd, 0, pcur);
  uint4 ocur = o_piece(0);
  float4 xcur[2];
  for (int k0 = 0; k0 < hd; k0 += 32) {
    stage(pcur);
    const uint4 a_bits = ocur;
    if (k0 + 32 < hd) {
      fetch(wo, hd, k0 + 32, pcur);
      ocur = o_piece(k0 + 32);
    } else if (wr) {
      fetch(wr, cin, 0, pcur);
      x_piece(0, xcur);
    }
    const bf16x8 a = __builtin_bit_cast(bf16x8, a_bits);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, *reinterpret_cast<const bf16x8 *>(&wst[16 * t + r][kq]),
                                                      acc[t], 0, 0, 0);
  }
  if (wr) {
    for (int k0 = 0; k0 < cin; k0 += 32) {
      stage(pcur);
      const f32x8v xf = {xcur[0].x, xcur[0].y, xcur[0].z, xcur[0].w, xcur[1].x, xcur[1].y, xcur[1].z, xcur[1].w};
      if (k0 + 32 < cin) {
        fetch(wr, cin, k0 + 32, pcur);
        x_piece(k0 + 32, xcur);
      }
      const bf16x8 a = __builtin_convertvector(xf, bf16x8);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        res[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, *reinterpret_cast<const bf16x8 *>(&wst[16 * t + r][kq]),
                                                        res[t], 0, 0, 0);
    }
  }
  if (e0 >= n) return;   // after the last barrier: nothing of this wavefront to write
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

// site_finish with both weight matrices resident in LDS for the whole
// launch (sizes fixed at compile time: the step's stage shapes).  A
// workgroup of kResWaves wavefronts stages Wo [C, HD] and Wr [C, CIN] once
// (rows padded by 8 elements, so the 16 lanes of an MFMA operand read
// spread over the banks), then takes row tiles of 16 kResWaves events
// blockIdx.x, blockIdx.x + gridDim.x, ... with no barrier between them:
// each wavefront loads all of its 16 rows' o and x pieces at once, then
// runs the same MFMA sequence and epilogue as site_finish_kernel (the same
// sums in the same order: the same bits).
constexpr int kResWaves = 8;
constexpr int kResRows = 16 * kResWaves;
template <int NT, int HD, int CIN, bool WR>
__global__ __launch_bounds__(64 * kResWaves) void site_finish_resident_kernel(
    const uint16_t *__restrict__ o, int64_t n, const uint16_t *__restrict__ wo, const float *__restrict__ x,
    const uint16_t *__restrict__ wr, const float *__restrict__ ln_w, const float *__restrict__ ln_b, float eps,
    float *__restrict__ y) {
  constexpr int C = 16 * NT;
  constexpr int PO = HD + 8, PR = CIN + 8;   // row pitches (elements)
  __shared__ __align__(16) uint16_t wlo[C * PO];
  __shared__ __align__(16) uint16_t wlr[WR ? C * PR : 8];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r = lane & 15, kq = 8 * (lane >> 4);
  for (int i = tid; i < C * (HD / 8); i += 64 * kResWaves) {
    const int rw = i / (HD / 8), c8 = i - rw * (HD / 8);
    *reinterpret_cast<uint4 *>(&wlo[rw * PO + 8 * c8]) = *reinterpret_cast<const uint4 *>(wo + rw * HD + 8 * c8);
  }
  if constexpr (WR) {
    for (int i = tid; i < C * (CIN / 8); i += 64 * kResWaves) {
      const int rw = i / (CIN / 8), c8 = i - rw * (CIN / 8);
      *reinterpret_cast<uint4 *>(&wlr[rw * PR + 8 * c8]) = *reinterpret_cast<const uint4 *>(wr + rw * CIN + 8 * c8);
    }
  }
  __syncthreads();
  const int64_t n_tiles = (n + kResRows - 1) / kResRows;
  for (int64_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
    const int64_t e0 = tile * kResRows + 16 * wv;
    if (e0 >= n) continue;   // wavefront-uniform; no barrier in the loop
    const int64_t row = min(e0 + r, n - 1);
    uint4 op[HD / 32];
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) op[s] = *reinterpret_cast<const uint4 *>(o + row * HD + 32 * s + kq);
    float4 xp[WR ? CIN / 32 : 1][2];
    if constexpr (WR) {
#pragma unroll
      for (int s = 0; s < CIN / 32; ++s) {
        xp[s][0] = *reinterpret_cast<const float4 *>(x + row * CIN + 32 * s + kq);
        xp[s][1] = *reinterpret_cast<const float4 *>(x + row * CIN + 32 * s + kq + 4);
      }
    }
    f32x4 acc[NT], res[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = res[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) {
      const bf16x8 a = __builtin_bit_cast(bf16x8, op[s]);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            a, *reinterpret_cast<const bf16x8 *>(&wlo[(16 * t + r) * PO + 32 * s + kq]), acc[t], 0, 0, 0);
    }
    if constexpr (WR) {
#pragma unroll
      for (int s = 0; s < CIN / 32; ++s) {
        const f32x8v xf = {xp[s][0].x, xp[s][0].y, xp[s][0].z, xp[s][0].w,
                           xp[s][1].x, xp[s][1].y, xp[s][1].z, xp[s][1].w};
        const bf16x8 a = __builtin_convertvector(xf, bf16x8);
#pragma unroll
        for (int t = 0; t < NT; ++t)
          res[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              a, *reinterpret_cast<const bf16x8 *>(&wlr[(16 * t + r) * PR + 32 * s + kq]), res[t], 0, 0, 0);
      }
    }
    float yv[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t ev = e0 + 4 * (lane >> 4) + i;
        const float rv = WR ? round_bf16(res[t][i]) : (ev < n ? x[ev * CIN + 16 * t + r] : 0.f);
        yv[t][i] = round_bf16(acc[t][i]) + rv;
      }
    float mean[4], rstd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float sm = 0.f;
#pragma unroll
      for (int t = 0; t < NT; ++t) sm += yv[t][i];
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) sm += __shfl_xor(sm, m);
      mean[i] = sm / static_cast<float>(C);
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
}

// Workgroups of the resident finish that fit the device at once (its LDS
// decides), for a grid that covers every row tile in one round or less.
template <int NT, int HD, int CIN, bool WR>
unsigned resident_grid(int64_t n) {
  static int per_cu = -1, cus = 0;
  if (per_cu < 0) {
    int dev = 0, b = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, site_finish_resident_kernel<NT, HD, CIN, WR>,
                                                     64 * kResWaves, 0) != hipSuccess)
      b = 1, cus = 256;
    per_cu = std::max(b, 1);
  }
  const int64_t tiles = (n + kResRows - 1) / kResRows;
  return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(tiles, static_cast<int64_t>(per_cu) * cus)));
}

}  // namespace
}  // namespace ssla

extern "C" int ssla_site_project(const float *x, int64_t n, int cin, const uint16_t *w, int hd, float gate_normalizer,
                                 uint16_t *q, uint16_t *k, uint16_t *v, float *g, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n >= 0 && cin > 0 && hd > 0 && gate_normalizer != 0.f,
                 "site_project: bad sizes n=%lld cin=%d hd=%d", (long long)n, cin, hd);
  if (cin % 32 != 0 || hd % 32 != 0) {
    set_error("site_project: needs cin and hd multiples of 32 (cin=%d hd=%d)", cin, hd);
    return SSLA_ERR_UNSUPPORTED;
  }
  SSLA_CHECK_ARG(n < (int64_t{1} << 31) * kRows, "site_project: too many rows");
  if (n == 0) return SSLA_OK;
  SSLA_CHECK_ARG(x && w && q && k && v && g, "site_project: null pointer");
  SSLA_CHECK_ARG(aligned(x, 16) && aligned(w, 16) && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) &&
                 aligned(g, 16), "site_project: x, w and the outputs must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // column chunks of 64 (32 when hd is not a multiple of 64): wider chunks
  // hold more accumulators than three wavefronts per SIMD can
  const int nto = hd % 64 == 0 ? 4 : 2;
  const dim3 grid(row_tiles(n), hd / (16 * nto));
  const float ig = 1.f / gate_normalizer;
  if (nto == 4)
    hipLaunchKernelGGL((site_project_kernel<4>), grid, dim3(64 * kWaves), 0, st, x, n, cin, w, hd, ig, q, k, v, g);
  else
    hipLaunchKernelGGL((site_project_kernel<2>), grid, dim3(64 * kWaves), 0, st, x, n, cin, w, hd, ig, q, k, v, g);
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
  // the step's stage shapes: weights resident in LDS
#define SITE_FINISH_RES(NTV, HDV, CINV, WRV)                                                                      \
  if (cout == 16 * NTV && hd == HDV && cin == CINV && (wr != nullptr) == WRV) {                                  \
    hipLaunchKernelGGL((site_finish_resident_kernel<NTV, HDV, CINV, WRV>),                                      \
                       dim3(resident_grid<NTV, HDV, CINV, WRV>(n)), dim3(64 * kResWaves), 0, st, o, n, wo, x, wr, \
                       ln_w, ln_b, eps, y);                                                                      \
    return launch_status("site_finish");                                                                         \
  }
  SITE_FINISH_RES(2, 128, 32, false) SITE_FINISH_RES(4, 128, 32, true) SITE_FINISH_RES(8, 128, 64, true)
  SITE_FINISH_RES(16, 128, 128, true)
#undef SITE_FINISH_RES
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

// ----------------------------------------------------------- detection head
// DetectionHead of the asynchronous step (ssla_amd.backbone; the YOLOX
// head's inference path, reference layers/yolox_head.py:183-230 forward,
// :234-256 decode) over all its levels in one launch.  Per cell of a level
// (rows of [batch * h * w]):
//   f = SiLU(BN(W_br x + b))      (the cls and reg branches side by side,
//                                   2 width channels; BN folded into
//                                   scale / shift by the caller)
//   p = W_pred f + b_pred          (reg 0-3, obj 4, classes 5.. : 16 rows,
//                                   zero where a prediction ignores a branch)
//   out = ((p0 + x) s, (p1 + y) s, exp(p2) s, exp(p3) s, p4, p5, ...)
// x is the fp32 grid [batch, c, h, w] rounded to bf16 (as the module's input
// is), the GEMMs run on bf16 operands with fp32 sums, the features are
// rounded to bf16 between the two GEMMs, and everything else is fp32 up to
// the bf16 output.
namespace ssla {
namespace {

constexpr int kHeadMaxW = 256;            // branch width
constexpr int kHeadF = 2 * kHeadMaxW;     // features per cell
constexpr int kHeadLdsRow = kHeadF + 8;   // bf16 elements per LDS row (16-byte pad)

struct HeadArgs {
  ssla_head_level lv[SSLA_HEAD_MAX_LEVELS];
  int tile0[SSLA_HEAD_MAX_LEVELS + 1];   // first workgroup of each level
  int anchor0[SSLA_HEAD_MAX_LEVELS];     // first anchor of each level
  int n_levels, batch, n_anchor, n_out, width;
};

// One workgroup per 16 cells of a level, 4 wavefronts: wavefront w computes
// the feature tiles t = w, w + 4, ... (16 features each) of the 16 cells,
// then the prediction GEMM's K range [128 w, 128 w + 128) of the features;
// the four partial predictions are summed through LDS and wavefront 0
// decodes and stores.  Splitting the features across the wavefronts (not
// the cells) keeps each wavefront's chain of dependent MFMAs short: the
// call is a few hundred workgroups with short chains instead of a few
// dozen with long ones.
constexpr int kHeadCells = 16;
__global__ __launch_bounds__(64 * kWaves) void detect_head_kernel(HeadArgs a, uint16_t *__restrict__ out) {
  __shared__ __align__(16) uint16_t feat[kHeadCells][kHeadLdsRow];
  __shared__ f32x4 part[kWaves][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 15, kq = 8 * (lane >> 4);
  int L = 0;
  while (L + 1 < a.n_levels && static_cast<int>(blockIdx.x) >= a.tile0[L + 1]) ++L;
  const ssla_head_level &lv = a.lv[L];
  const int hw = lv.h * lv.w, n_cell = a.batch * hw;
  const int c0 = (static_cast<int>(blockIdx.x) - a.tile0[L]) * kHeadCells;   // this workgroup's first cell
  const int F = 2 * a.width;
  // ---- branches: 16 cells x this wavefront's feature tiles, K = c in steps of 32
  {
    const int cell = c0 + r;
    const bool ok = cell < n_cell;
    const int b = ok ? cell / hw : 0, rem = ok ? cell - b * hw : 0;
    const float *xb = lv.grid + static_cast<int64_t>(b) * lv.c * hw + rem;
    constexpr int NT = kHeadF / 16 / kWaves;   // tiles per wavefront
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < lv.c; k0 += 32) {
      f32x8v xv;
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[e] = ok ? xb[static_cast<int64_t>(k0 + kq + e) * hw] : 0.f;
      const bf16x8 av = __builtin_convertvector(xv, bf16x8);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int tile = kWaves * t + wv;
        if (16 * tile < F)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bf16_piece(lv.w_br, 16 * tile + r, lv.c, k0 + kq, true),
                                                          acc[t], 0, 0, 0);
      }
    }
    // f = SiLU(acc scale + shift), rounded to bf16, into the features' rows
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int tile = kWaves * t + wv;
      if (16 * tile >= F) continue;
      const int col = 16 * tile + r;
      const float sc = lv.br_scale[col], sh = lv.br_shift[col];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float y = fmaf(acc[t][i], sc, sh);
        const float f = y / (1.f + expf(-y));
        feat[4 * (lane >> 4) + i][col] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
      }
    }
  }
  __syncthreads();
  // ---- predictions: 16 cells x 16 outputs, this wavefront's quarter of K = F
  {
    f32x4 p = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 32 * wv; k0 < F; k0 += 32 * kWaves) {   // F is a multiple of 32 (host check)
      const bf16x8 av = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(&feat[r][k0 + kq]));
      p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bf16_piece(lv.w_pred, r, F, k0 + kq, true), p, 0, 0, 0);
    }
    part[wv][lane] = p;
  }
  __syncthreads();
  if (wv != 0) return;
  f32x4 p = part[0][lane];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) p += part[w][lane];
  const int j = r;   // output column
  if (j >= a.n_out) return;
  const float s = static_cast<float>(lv.stride), bj = lv.b_pred[j];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int cell = c0 + 4 * (lane >> 4) + i;
    if (cell >= n_cell) continue;
    const int b = cell / hw, rem = cell - b * hw;
    float v = p[i] + bj;
    if (j == 0) v = (v + static_cast<float>(rem % lv.w)) * s;
    else if (j == 1) v = (v + static_cast<float>(rem / lv.w)) * s;
    else if (j < 4) v = expf(v) * s;
    const int64_t o = (static_cast<int64_t>(b) * a.n_anchor + a.anchor0[L] + rem) * a.n_out + j;
    out[o] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  }
}

}  // namespace
}  // namespace ssla

extern "C" int ssla_detect_head(const ssla_head_level *levels, int n_levels, int batch, int n_out, int width,
                                uint16_t *out, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(levels && out && n_levels > 0 && n_levels <= SSLA_HEAD_MAX_LEVELS && batch > 0,
                 "detect_head: bad arguments (levels=%d batch=%d)", n_levels, batch);
  if (width <= 0 || width > kHeadMaxW || width % 16 != 0 || n_out < 5 || n_out > 16) {
    set_error("detect_head: needs a branch width that is a multiple of 16 up to %d and 5..16 outputs "
              "(width=%d n_out=%d)", kHeadMaxW, width, n_out);
    return SSLA_ERR_UNSUPPORTED;
  }
  HeadArgs a{};
  a.n_levels = n_levels;
  a.batch = batch;
  a.n_out = n_out;
  a.width = width;
  int64_t tiles = 0, anchors = 0;
  for (int l = 0; l < n_levels; ++l) {
    const ssla_head_level &lv = levels[l];
    SSLA_CHECK_ARG(lv.grid && lv.w_br && lv.br_scale && lv.br_shift && lv.w_pred && lv.b_pred,
                   "detect_head: null pointer in level %d", l);
    SSLA_CHECK_ARG(lv.h > 0 && lv.w > 0 && lv.stride > 0, "detect_head: bad level %d", l);
    if (lv.c <= 0 || lv.c % 32 != 0) {
      set_error("detect_head: level %d has %d input channels (a multiple of 32 needed)", l, lv.c);
      return SSLA_ERR_UNSUPPORTED;
    }
    SSLA_CHECK_ARG(aligned(lv.w_br, 16) && aligned(lv.w_pred, 16), "detect_head: weights must be 16-byte aligned");
    a.lv[l] = lv;
    a.tile0[l] = static_cast<int>(tiles);
    a.anchor0[l] = static_cast<int>(anchors);
    const int64_t cells = static_cast<int64_t>(batch) * lv.h * lv.w;
    tiles += (cells + kHeadCells - 1) / kHeadCells;
    anchors += static_cast<int64_t>(lv.h) * lv.w;
    SSLA_CHECK_ARG(tiles < (int64_t{1} << 30) && anchors * batch * n_out < (int64_t{1} << 31),
                   "detect_head: too many cells");
  }
  a.tile0[n_levels] = static_cast<int>(tiles);
  a.n_anchor = static_cast<int>(anchors);
  hipLaunchKernelGGL(detect_head_kernel, dim3(static_cast<unsigned>(tiles)), dim3(64 * kWaves), 0,
                     static_cast<hipStream_t>(stream), a, out);
  return launch_status("detect_head");
}

// ------------------------------------------------------- the whole block
// SiteGLABlock.forward on the sites of one window in one call: the sequence
// offsets and state rows of the groups, ssla_site_project, the per-site
// recurrence (ssla_gla_recurrent_fwd with state_idx, the states updated in
// place) and ssla_site_finish.
namespace ssla {
namespace {
constexpr int kKeyThreads = 1024, kKeyPer = 8;

// cu[0..G] = exclusive prefix of the group lengths (cu[G] the total) and
// sites[g] = (b * grid_h + h) * grid_w + w, in one workgroup: chunks of
// kKeyThreads * kKeyPer lengths in turn, each scanned across the
// wavefronts through LDS, the running total carried between chunks.
__global__ __launch_bounds__(kKeyThreads) void site_keys_kernel(const int64_t *__restrict__ len,
                                                                const int64_t *__restrict__ gb,
                                                                const int64_t *__restrict__ gh,
                                                                const int64_t *__restrict__ gw, int64_t G, int grid_h,
                                                                int grid_w, int64_t *__restrict__ cu,
                                                                int32_t *__restrict__ sites) {
  __shared__ int64_t wsum[kKeyThreads / 64];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int64_t carry = 0;
  for (int64_t base = 0; base < G; base += static_cast<int64_t>(kKeyThreads) * kKeyPer) {
    int64_t v[kKeyPer];
    int64_t s = 0;
#pragma unroll
    for (int e = 0; e < kKeyPer; ++e) {
      const int64_t i = base + static_cast<int64_t>(t) * kKeyPer + e;
      v[e] = i < G ? len[i] : 0;
      s += v[e];
    }
    int64_t x = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int64_t run = carry + x - s, total = carry;
    for (int j = 0; j < kKeyThreads / 64; ++j) {
      if (j < w) run += wsum[j];
      total += wsum[j];
    }
#pragma unroll
    for (int e = 0; e < kKeyPer; ++e) {
      const int64_t i = base + static_cast<int64_t>(t) * kKeyPer + e;
      if (i < G) cu[i] = run;
      run += v[e];
    }
    carry = total;
    __syncthreads();   // wsum is rewritten by the next chunk
  }
  if (t == 0) cu[G] = carry;
  for (int64_t g = t; g < G; g += kKeyThreads)
    sites[g] = static_cast<int32_t>((gb[g] * grid_h + gh[g]) * grid_w + gw[g]);
}

struct BlockWs {
  uint16_t *q, *k, *v, *o;
  float *g;
  int64_t *cu;
  int32_t *sites;
  void *rec;
  size_t rec_bytes, total;
};
BlockWs block_layout(void *ws, int64_t n, int64_t G, int heads, int head_dim) {
  auto up = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
  char *b = static_cast<char *>(ws);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    void *p = b ? b + off : nullptr;
    off = up(off + std::max<size_t>(bytes, 1));
    return p;
  };
  const size_t rows = static_cast<size_t>(n) * heads * head_dim;
  BlockWs L;
  L.q = static_cast<uint16_t *>(take(2 * rows));
  L.k = static_cast<uint16_t *>(take(2 * rows));
  L.v = static_cast<uint16_t *>(take(2 * rows));
  L.o = static_cast<uint16_t *>(take(2 * rows));
  L.g = static_cast<float *>(take(4 * rows));
  L.cu = static_cast<int64_t *>(take(8 * (G + 1)));
  L.sites = static_cast<int32_t *>(take(4 * G));
  L.rec_bytes = ssla_gla_recurrent_workspace_size(static_cast<int>(std::min<int64_t>(G, 0x7fffffff)), n, heads,
                                                  head_dim, head_dim);
  L.rec = L.rec_bytes ? take(L.rec_bytes) : nullptr;
  L.total = off;
  return L;
}
}  // namespace
}  // namespace ssla

extern "C" size_t ssla_site_gla_block_workspace_size(int64_t n, int64_t G, int heads, int head_dim) {
  if (n < 0 || G < 0 || heads <= 0 || head_dim <= 0) return 0;
  return ssla::block_layout(nullptr, n, G, heads, head_dim).total;
}

extern "C" int ssla_site_gla_block(const float *x, int64_t n, int cin, const int64_t *lengths, const int64_t *gr_batch,
                                   const int64_t *gr_h, const int64_t *gr_w, int64_t G, int grid_h, int grid_w,
                                   float *state, int n_sites, int heads, int head_dim, const uint16_t *w_qkvg,
                                   float gate_normalizer, float scale, const uint16_t *w_o, const uint16_t *w_r,
                                   const float *ln_w, const float *ln_b, float eps, int cout, float *y,
                                   int32_t *status, void *workspace, size_t workspace_bytes, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n >= 0 && G >= 0 && G < 0x7fffffff && cin > 0 && cout > 0 && heads > 0 && head_dim > 0 &&
                     grid_h > 0 && grid_w > 0 && n_sites > 0,
                 "site_gla_block: bad sizes");
  const BlockWs L = block_layout(workspace, n, G, heads, head_dim);
  if (!workspace || workspace_bytes < L.total) {
    set_error("site_gla_block: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  if (n == 0 || G == 0) return SSLA_OK;
  SSLA_CHECK_ARG(lengths && gr_batch && gr_h && gr_w && state, "site_gla_block: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int hd = heads * head_dim;
  hipLaunchKernelGGL(site_keys_kernel, dim3(1), dim3(kKeyThreads), 0, st, lengths, gr_batch, gr_h, gr_w, G, grid_h,
                     grid_w, L.cu, L.sites);
  int s = ssla_site_project(x, n, cin, w_qkvg, hd, gate_normalizer, L.q, L.k, L.v, L.g, stream);
  if (s) return s;
  s = ssla_gla_recurrent_fwd(L.q, L.k, L.v, L.g, SSLA_F32, L.cu, static_cast<int>(G), n, heads, head_dim, head_dim,
                             scale, state, L.o, state, L.sites, n_sites, status, SSLA_BF16, L.rec, L.rec_bytes,
                             stream);
  if (s) return s;
  return ssla_site_finish(L.o, n, hd, w_o, x, cin, w_r, ln_w, ln_b, eps, cout, y, stream);
}
