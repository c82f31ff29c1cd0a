// Fused MosAttention forward on gfx950 (inference path).
//
// Reference: layers/mos_attention.py:75-140 after scatter_group_events_to_patch
// (utils/async_utils.py:125-240), with _apply_scatter_proj / _apply_gather_proj
// (mos_attention.py:148-167), scan (ops/common/scan.py:20-43) and
// gather_patch_events_to_group (utils/async_utils.py:243-264).  Per patch row
// r (rows of one patch consecutive, in time order; src[r] the pixel event,
// pos[r] its kernel position):
//   x   = Ws[pos] e[src]                  (scatter projection)
//   q   = Wq x,  v = Wv x,  a = sigmoid(Wg x)
//   h_r = a_r h_(r-1) + v_r               (h = 0 before each patch)
//   o_r = Wgp[pos] (Wo (q h))             (o_proj, then gather projection)
// and per pixel event e:
//   y_e = LayerNorm(sum over the copies r of e of o_r + (Win e or e)).
//
// Kernels:
// * mos_mark_starts / mos_dst_fill -- patch-start flags from the patch
//   lengths, and the inverse of the row -> (event, position) map:
//   dst[e * A + pos] = r (each pair occurs at most once), so the sum over an
//   event's copies needs no sort.
// * mos_patch_kernel -- one lane per patch row: the projections run in
//   registers with the weights in LDS (position-dependent matrices padded so
//   that lanes reading different positions hit different banks), the
//   recurrence is a segmented scan of the pairs (a, v) across the wavefront
//   (combine (A1, B1) then (A2, B2) = (A1 A2, A2 B1 + B2), restarted at patch
//   starts), carried from one 64-row window to the next.  Each wavefront
//   owns a window of rows [k L, (k + 1) L) shifted to patch boundaries: it
//   starts at the first patch start at or after k L and finishes the patch
//   that crosses (k + 1) L, so no patch is split between wavefronts.
// * mos_event_kernel -- one lane per pixel event: the copies summed in
//   increasing patch order (decreasing kernel position), the residual (or its
//   input projection) added, then LayerNorm over the hidden channels.
// All arithmetic is fp32.
#include <cstring>
#include <rocprim/rocprim.hpp>

#include "common.h"

namespace ssla {
namespace {

constexpr int kThreads = 256;
constexpr int kWin = 256;       // rows per wavefront window (before the shift to patch boundaries)
constexpr int kMaxPos = 49;     // kernel positions (up to 7 x 7)
constexpr size_t kMaxLds = 64 * 1024;   // weights held in LDS per workgroup

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
inline unsigned grid_for(int64_t n) {
  return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((n + kThreads - 1) / kThreads, 1 << 20)));
}
#define MOS_GRID_STRIDE(i, n)                                                                   \
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < (n);      \
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)

struct MosWs {
  int64_t *cu;       // [n_patch + 1] exclusive scan of the patch lengths
  uint8_t *start;    // [R] 1 at the first row of every patch
  int32_t *dst;      // [E * A] row of (event, position), or -1
  float *orow;       // [R + 1, HP] projected rows, row R zero
  float *wfold;      // folded weights (3 A scatter-side + A gather-side matrices)
  void *tmp;
  size_t tmp_bytes, total;
};

size_t scan_bytes(int64_t n) {
  size_t tb = 0;
  (void)rocprim::exclusive_scan(nullptr, tb, static_cast<int64_t *>(nullptr), static_cast<int64_t *>(nullptr),
                          static_cast<int64_t>(0), static_cast<size_t>(std::max<int64_t>(n, 1)),
                          rocprim::plus<int64_t>());
  return tb;
}

MosWs mos_layout(void *base, int64_t E, int A, int64_t R, int64_t n_patch, int CP, int HP) {
  char *b = static_cast<char *>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char *p = b ? b + off : nullptr;
    off = align256(off + std::max<size_t>(bytes, 1));
    return p;
  };
  MosWs w;
  w.cu = reinterpret_cast<int64_t *>(take(sizeof(int64_t) * (n_patch + 1)));
  w.start = reinterpret_cast<uint8_t *>(take(static_cast<size_t>(R)));
  w.dst = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * static_cast<size_t>(E) * A));
  w.orow = reinterpret_cast<float *>(take(sizeof(float) * static_cast<size_t>(R + 1) * HP));   // + zero row
  w.wfold = reinterpret_cast<float *>(
      take(sizeof(float) * (3 * static_cast<size_t>(A) * (HP * CP + 4) + static_cast<size_t>(A) * (HP * HP + 4))));
  w.tmp_bytes = scan_bytes(n_patch);
  w.tmp = take(w.tmp_bytes);
  w.total = off;
  return w;
}

__global__ void mos_fill_u8(uint8_t *p, int64_t n) { MOS_GRID_STRIDE(i, n) p[i] = 0; }
__global__ void mos_fill_i32(int32_t *p, int64_t n, int32_t v) { MOS_GRID_STRIDE(i, n) p[i] = v; }

// start[cu[p]] = 1 for every patch (empty patches mark the next patch's
// first row, which is a start anyway).
__global__ void mos_mark_starts(const int64_t *__restrict__ cu, int64_t n_patch, int64_t R,
                                uint8_t *__restrict__ start) {
  if (blockIdx.x == 0 && threadIdx.x == 0 && R > 0) start[0] = 1;   // rows before the first patch: none
  MOS_GRID_STRIDE(p, n_patch) {
    const int64_t r = cu[p];
    if (r >= 0 && r < R) start[r] = 1;
  }
}

__global__ void mos_dst_fill(const int64_t *__restrict__ src, const int64_t *__restrict__ pos, int64_t R,
                             int64_t E, int A, int32_t *__restrict__ dst) {
  MOS_GRID_STRIDE(r, R) {
    const int64_t s = src[r], a = pos[r];
    if (s >= 0 && s < E && a >= 0 && a < A) dst[s * A + a] = static_cast<int32_t>(r);
  }
}

// LDS weight layout (floats): position-dependent matrices are padded by 4
// floats each so that lanes on different positions read different banks.
template <int CP, int HP>
struct MosW {
  static constexpr int kS = HP * CP + 4;   // scatter matrix stride
  static constexpr int kG = HP * HP + 4;   // gather matrix stride
  static constexpr int kU = HP * HP;       // uniform matrices
  static size_t bytes(int As, int Ag) { return sizeof(float) * (static_cast<size_t>(As) * kS + Ag * kG + 4 * kU); }
  // folded: Wq Ws[a], Wv Ws[a], Wg Ws[a] (stride kS) and Wgp[a] Wo (stride kG)
  __host__ __device__ static size_t fold_floats(int As, int Ag) { return 3 * static_cast<size_t>(As) * kS + static_cast<size_t>(Ag) * kG; }
  static size_t fold_bytes(int As, int Ag) { return sizeof(float) * fold_floats(As, Ag); }
};

// The folded matrices in their LDS layout (zero-padded), once per call:
// q = (Wq Ws[a]) e, v = (Wv Ws[a]) e, g = (Wg Ws[a]) e and o = (Wgp[a] Wo)(q h)
// take 3 cin hid + hid^2 FMAs per row instead of 4 hid^2 + cin hid + hid^2.
template <int CP, int HP>
__global__ void mos_fold_weights(const float *__restrict__ ws, int As, const float *__restrict__ wq,
                                 const float *__restrict__ wv, const float *__restrict__ wg,
                                 const float *__restrict__ wo, const float *__restrict__ wgp, int Ag, int cin, int hid,
                                 float *__restrict__ out) {
  typedef MosW<CP, HP> L;
  const int64_t n_s = 3 * static_cast<int64_t>(As) * L::kS, n = static_cast<int64_t>(L::fold_floats(As, Ag));
  MOS_GRID_STRIDE(i, n) {
    float acc = 0.f;
    if (i < n_s) {
      const int m = static_cast<int>(i / (As * L::kS));
      const int rem = static_cast<int>(i % (As * L::kS)), a = rem / L::kS, o = rem % L::kS;
      const int j = o / CP, c = o % CP;
      if (o < HP * CP && j < hid && c < cin) {
        const float *w = m == 0 ? wq : m == 1 ? wv : wg;
        for (int k = 0; k < hid; ++k) acc = fmaf(w[j * hid + k], ws[(static_cast<int64_t>(a) * hid + k) * cin + c], acc);
      }
    } else {
      const int i2 = static_cast<int>(i - n_s), a = i2 / L::kG, o = i2 % L::kG;
      const int j = o / HP, c = o % HP;
      if (o < HP * HP && j < hid && c < hid)
        for (int k = 0; k < hid; ++k) acc = fmaf(wgp[(static_cast<int64_t>(a) * hid + j) * hid + k], wo[k * hid + c], acc);
    }
    out[i] = acc;
  }
}

// Fill the padded LDS copy of the weights (zeros outside cin x hid).
template <int CP, int HP>
__device__ void load_weights(float *sw, const float *ws, int As, const float *wq, const float *wv, const float *wg,
                             const float *wo, const float *wgp, int Ag, int cin, int hid) {
  typedef MosW<CP, HP> L;
  float *s_s = sw, *s_g = sw + As * L::kS, *s_u = s_g + Ag * L::kG;
  const int n_s = As * L::kS, n_g = Ag * L::kG;
  for (int i = threadIdx.x; i < n_s; i += blockDim.x) {
    const int a = i / L::kS, o = i % L::kS, j = o / CP, c = o % CP;
    s_s[i] = (o < HP * CP && j < hid && c < cin) ? ws[(static_cast<int64_t>(a) * hid + j) * cin + c] : 0.f;
  }
  for (int i = threadIdx.x; i < n_g; i += blockDim.x) {
    const int a = i / L::kG, o = i % L::kG, j = o / HP, c = o % HP;
    s_g[i] = (o < HP * HP && j < hid && c < hid) ? wgp[(static_cast<int64_t>(a) * hid + j) * hid + c] : 0.f;
  }
  for (int i = threadIdx.x; i < 4 * L::kU; i += blockDim.x) {
    const int m = i / L::kU, o = i % L::kU, j = o / HP, c = o % HP;
    const float *src = m == 0 ? wq : m == 1 ? wv : m == 2 ? wg : wo;
    s_u[i] = (j < hid && c < hid) ? src[j * hid + c] : 0.f;
  }
}

// First row >= x that starts a patch (R if none): 64 flags per step.
__device__ __forceinline__ int64_t next_start(const uint8_t *__restrict__ start, int64_t x, int64_t R, int lane) {
  for (int64_t y = x; y < R; y += 64) {
    const int64_t r = y + lane;
    const bool f = r < R && start[r] != 0;
    const unsigned long long m = __ballot(f);
    if (m) return y + __builtin_ctzll(m);
  }
  return R;
}

// Dot product of an LDS weight row (16-byte aligned when N % 4 == 0, 8-byte
// when N % 2 == 0) with x, in column order: one 16-byte LDS read per four
// FMAs.
template <int N>
__device__ __forceinline__ float dot_lds(const float *row, const float (&x)[N]) {
  float acc = 0.f;
  if constexpr (N % 4 == 0) {
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
#pragma unroll
    for (int c = 0; c < N; c += 4) {
      const float4 w = r4[c / 4];
      acc = fmaf(w.x, x[c], acc);
      acc = fmaf(w.y, x[c + 1], acc);
      acc = fmaf(w.z, x[c + 2], acc);
      acc = fmaf(w.w, x[c + 3], acc);
    }
  } else if constexpr (N % 2 == 0) {
    const float2 *r2 = reinterpret_cast<const float2 *>(row);
#pragma unroll
    for (int c = 0; c < N; c += 2) {
      const float2 w = r2[c / 2];
      acc = fmaf(w.x, x[c], acc);
      acc = fmaf(w.y, x[c + 1], acc);
    }
  } else {
#pragma unroll
    for (int c = 0; c < N; ++c) acc = fmaf(row[c], x[c], acc);
  }
  return acc;
}

// Index, position and start flag of patch row r (r >= re: a start with
// index 0, which keeps every later load in bounds).
struct RowIdx {
  int64_t s;
  int p, flag;
};
__device__ __forceinline__ void fetch_idx(RowIdx &ix, const int64_t *__restrict__ src,
                                          const int64_t *__restrict__ pos, const uint8_t *__restrict__ start,
                                          int64_t r, int64_t re, int64_t E, int A) {
  ix.s = 0;
  ix.p = 0;
  ix.flag = 1;
  if (r < re) {
    ix.s = min(max(src[r], (int64_t)0), E - 1);
    ix.p = static_cast<int>(min(max(pos[r], (int64_t)0), static_cast<int64_t>(A - 1)));
    ix.flag = start[r] != 0;
  }
}

// Event row s (cin values, zero-padded to CP): 16-byte loads when the row
// is exactly CP wide and CP is a multiple of 4 (rows then stay 16-byte
// aligned), else element loads.
template <int CP>
__device__ __forceinline__ void fetch_row(float (&e)[CP], const float *__restrict__ ev, int64_t s, int cin) {
  if (CP % 4 == 0 && cin == CP) {
    const float4 *p = reinterpret_cast<const float4 *>(ev + s * CP);
#pragma unroll
    for (int c = 0; c < CP; c += 4) {
      const float4 t = p[c / 4];
      e[c] = t.x;
      e[c + 1] = t.y;
      e[c + 2] = t.z;
      e[c + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < CP; ++c) e[c] = c < cin ? ev[s * cin + c] : 0.f;
  }
}

// One step of the segmented scan: every lane combines with the value that
// the DPP control CTRL brings from an earlier lane, (A, B) of that lane then
// this one: (A_s A, A B_s + B), unless a patch starts inside this lane's
// range (F).  Lanes without a source (outside row_mask, or before the
// shift's reach in their row) receive the identity (1, 0, no start).
template <int CTRL, int ROWS, int HP>
__device__ __forceinline__ void seg_scan_step(float (&A)[HP], float (&B)[HP], int &F) {
  const int Fs = __builtin_amdgcn_update_dpp(0, F, CTRL, ROWS, 0xf, false);
  const bool take = !F;
#pragma unroll
  for (int j = 0; j < HP; ++j) {
    const float As = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 1.f), __builtin_bit_cast(int, A[j]), CTRL, ROWS,
                                           0xf, false));
    const float Bs = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, B[j]), CTRL, ROWS, 0xf, false));
    if (take) {
      B[j] = fmaf(A[j], Bs, B[j]);
      A[j] = A[j] * As;
    }
  }
  F |= Fs;
}

// Segmented inclusive scan of the pairs (A, B) over the 64 lanes (lane =
// row of the window, in order), restarted where a lane's flag is set: shifts
// by 1, 2, 4, 8 inside each 16-lane row (DPP row_shr), then lane 15 of rows
// 0 and 2 into rows 1 and 3 (row_bcast:15) and lane 31 into rows 2 and 3
// (row_bcast:31).  All on the VALU (no LDS permutes).
template <int HP>
__device__ __forceinline__ void seg_scan_dpp(float (&A)[HP], float (&B)[HP], int &F) {
  seg_scan_step<0x111, 0xf, HP>(A, B, F);   // row_shr:1
  seg_scan_step<0x112, 0xf, HP>(A, B, F);   // row_shr:2
  seg_scan_step<0x114, 0xf, HP>(A, B, F);   // row_shr:4
  seg_scan_step<0x118, 0xf, HP>(A, B, F);   // row_shr:8
  seg_scan_step<0x142, 0xa, HP>(A, B, F);   // row_bcast:15 into rows 1, 3
  seg_scan_step<0x143, 0xc, HP>(A, B, F);   // row_bcast:31 into rows 2, 3
}

template <int CP, int HP, bool FOLD>
__global__ __launch_bounds__(kThreads) void mos_patch_kernel(
    const float *__restrict__ ev, int64_t E, int cin, int hid, const int64_t *__restrict__ src,
    const int64_t *__restrict__ pos, int64_t R, const uint8_t *__restrict__ start, int A,
    const float *__restrict__ ws, int As, const float *__restrict__ wq, const float *__restrict__ wv,
    const float *__restrict__ wg, const float *__restrict__ wo, const float *__restrict__ wgp, int Ag,
    const float *__restrict__ wfold, float *__restrict__ orow) {
  typedef MosW<CP, HP> L;
  extern __shared__ float4 sw4[];   // 16-byte aligned: every matrix stride is a multiple of 4 floats
  float *sw = reinterpret_cast<float *>(sw4);
  if constexpr (FOLD) {
    const int n4 = static_cast<int>(L::fold_floats(As, Ag) / 4);
    const float4 *src4 = reinterpret_cast<const float4 *>(wfold);
    for (int i = threadIdx.x; i < n4; i += blockDim.x) sw4[i] = src4[i];
  } else {
    load_weights<CP, HP>(sw, ws, As, wq, wv, wg, wo, wgp, Ag, cin, hid);
  }
  __syncthreads();
  // unfolded layout
  const float *s_s = sw, *s_g = sw + As * L::kS, *s_u = s_g + Ag * L::kG;
  const float *s_q = s_u, *s_v = s_u + L::kU, *s_a = s_u + 2 * L::kU, *s_o = s_u + 3 * L::kU;
  // folded layout
  const float *f_q = sw, *f_v = sw + As * L::kS, *f_g = sw + 2 * As * L::kS, *f_o = sw + 3 * As * L::kS;

  const int lane = threadIdx.x & 63;
  const int64_t n_win = (R + kWin - 1) / kWin;
  const int64_t wave0 = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * (kThreads / 64);
  for (int64_t k = wave0; k < n_win; k += n_waves) {
    const int64_t rs = next_start(start, k * kWin, R, lane);
    const int64_t re = next_start(start, std::min<int64_t>((k + 1) * kWin, R), R, lane);
    float carry[HP];
#pragma unroll
    for (int j = 0; j < HP; ++j) carry[j] = 0.f;
    // two-stage prefetch: row indices two windows ahead, event rows one
    // window ahead (their address needs the index), compute on the current
    RowIdx i0, i1;
    float e0[CP];
    fetch_idx(i0, src, pos, start, rs + lane, re, E, A);
    fetch_row<CP>(e0, ev, i0.s, cin);
    fetch_idx(i1, src, pos, start, rs + 64 + lane, re, E, A);
    for (int64_t b = rs; b < re; b += 64) {
      // weights are re-read from LDS each window (broadcast reads) rather
      // than hoisted into registers, which would cost all the occupancy
      asm volatile("" ::: "memory");
      const int64_t r = b + lane;
      const bool valid = r < re;
      float en[CP];
      RowIdx i2;
      if (b + 64 < re) {
        fetch_row<CP>(en, ev, i1.s, cin);
      } else {
#pragma unroll
        for (int c = 0; c < CP; ++c) en[c] = 0.f;
      }
      fetch_idx(i2, src, pos, start, b + 128 + lane, re, E, A);
      const int flag = i0.flag;
      const int ps = As > 1 ? i0.p : 0, pg = Ag > 1 ? i0.p : 0;
      float e[CP];
#pragma unroll
      for (int c = 0; c < CP; ++c) e[c] = e0[c];
      // scatter projection, q, v, gate
      float q[HP], A_[HP], B_[HP];
      if constexpr (FOLD) {
        const int off = ps * L::kS;
#pragma unroll
        for (int j = 0; j < HP; ++j) {
          q[j] = dot_lds<CP>(f_q + off + j * CP, e);
          B_[j] = dot_lds<CP>(f_v + off + j * CP, e);
          const float ag = dot_lds<CP>(f_g + off + j * CP, e);
          // sigmoid on the transcendental unit (exp2 and reciprocal, ~1 ulp each)
          A_[j] = __builtin_amdgcn_rcpf(1.f + fast_exp2(-ag * kLog2e));
        }
      } else {
        float x[HP];
        const float *m = s_s + ps * L::kS;
#pragma unroll
        for (int j = 0; j < HP; ++j) x[j] = dot_lds<CP>(m + j * CP, e);
#pragma unroll
        for (int j = 0; j < HP; ++j) {
          q[j] = dot_lds<HP>(s_q + j * HP, x);
          B_[j] = dot_lds<HP>(s_v + j * HP, x);
          const float ag = dot_lds<HP>(s_a + j * HP, x);
          A_[j] = __builtin_amdgcn_rcpf(1.f + fast_exp2(-ag * kLog2e));
        }
      }
      // segmented inclusive scan of (A, B) across the wavefront
      int F = flag;
      seg_scan_dpp<HP>(A_, B_, F);
      // rows whose patch started before this window continue the carry
      float hq[HP];
#pragma unroll
      for (int j = 0; j < HP; ++j) {
        const float h = F ? B_[j] : fmaf(A_[j], carry[j], B_[j]);
        carry[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, h), 63));
        hq[j] = q[j] * h;
      }
      // o_proj, then the gather projection (folded: one product)
      float o[HP];
      if constexpr (FOLD) {
#pragma unroll
        for (int j = 0; j < HP; ++j) o[j] = hq[j];
      } else {
#pragma unroll
        for (int j = 0; j < HP; ++j) o[j] = dot_lds<HP>(s_o + j * HP, hq);
      }
      if (valid) {
        const float *m = (FOLD ? f_o : s_g) + pg * L::kG;
        float *dst = orow + r * HP;
#pragma unroll
        for (int j = 0; j < HP; j += 4) {
          float4 y;
          float *yy = reinterpret_cast<float *>(&y);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            yy[u] = j + u < HP ? dot_lds<HP>(m + (j + u) * HP, o) : 0.f;
          }
          *reinterpret_cast<float4 *>(dst + j) = y;
        }
      }
      i0 = i1;
      i1 = i2;
#pragma unroll
      for (int c = 0; c < CP; ++c) e0[c] = en[c];
    }
  }
}

// One lane per pixel event: sum of its copies, residual, LayerNorm.
template <int CP, int HP>
__global__ __launch_bounds__(kThreads) void mos_event_kernel(
    const float *__restrict__ ev, int64_t E, int cin, int hid, int A, const int32_t *__restrict__ dst,
    const float *__restrict__ orow, int64_t R, const float *__restrict__ win, const float *__restrict__ ln_w,
    const float *__restrict__ ln_b, float eps, float *__restrict__ out) {
  __shared__ float s_in[HP * CP], s_w[HP], s_b[HP];
  for (int i = threadIdx.x; i < HP * CP; i += blockDim.x) {
    const int j = i / CP, c = i % CP;
    s_in[i] = (win && j < hid && c < cin) ? win[j * cin + c] : 0.f;
  }
  for (int i = threadIdx.x; i < HP; i += blockDim.x) {
    s_w[i] = i < hid ? ln_w[i] : 0.f;
    s_b[i] = i < hid ? ln_b[i] : 0.f;
  }
  __syncthreads();
  MOS_GRID_STRIDE(e, E) {
    asm volatile("" ::: "memory");   // keep the weights in LDS, not in registers
    float y[HP];
#pragma unroll
    for (int j = 0; j < HP; ++j) y[j] = 0.f;
    // copies in decreasing kernel position, three at a time with every row
    // load issued before the adds (a missing copy reads the zero row R)
    for (int a0 = A - 1; a0 >= 0; a0 -= 3) {
      const float *p[3];
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        const int a = a0 - u;
        const int32_t r = a >= 0 ? dst[e * A + a] : -1;
        p[u] = orow + (r >= 0 && r < R ? static_cast<int64_t>(r) : R) * HP;
      }
      float4 t[3][HP / 4];
#pragma unroll
      for (int u = 0; u < 3; ++u)
#pragma unroll
        for (int j = 0; j < HP / 4; ++j) t[u][j] = reinterpret_cast<const float4 *>(p[u])[j];
#pragma unroll
      for (int u = 0; u < 3; ++u)
#pragma unroll
        for (int j = 0; j < HP / 4; ++j) {
          y[4 * j] += t[u][j].x;
          y[4 * j + 1] += t[u][j].y;
          y[4 * j + 2] += t[u][j].z;
          y[4 * j + 3] += t[u][j].w;
        }
    }
    float x[CP];
    fetch_row<CP>(x, ev, e, cin);
    if (win) {
#pragma unroll
      for (int j = 0; j < HP; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CP; ++c) acc = fmaf(s_in[j * CP + c], x[c], acc);
        y[j] += acc;
      }
    } else {
#pragma unroll
      for (int j = 0; j < HP; ++j) y[j] += (j < CP && j < cin) ? x[j < CP ? j : 0] : 0.f;
    }
    float mean = 0.f;
#pragma unroll
    for (int j = 0; j < HP; ++j) mean += j < hid ? y[j] : 0.f;
    mean /= static_cast<float>(hid);
    float var = 0.f;
#pragma unroll
    for (int j = 0; j < HP; ++j) {
      const float d = y[j] - mean;
      var += j < hid ? d * d : 0.f;
    }
    var /= static_cast<float>(hid);
    const float rstd = 1.f / sqrtf(var + eps);
    if (HP % 4 == 0 && hid == HP) {
      float4 *po = reinterpret_cast<float4 *>(out + e * HP);
#pragma unroll
      for (int j = 0; j < HP; j += 4)
        po[j / 4] = make_float4((y[j] - mean) * rstd * s_w[j] + s_b[j], (y[j + 1] - mean) * rstd * s_w[j + 1] + s_b[j + 1],
                                (y[j + 2] - mean) * rstd * s_w[j + 2] + s_b[j + 2],
                                (y[j + 3] - mean) * rstd * s_w[j + 3] + s_b[j + 3]);
    } else {
#pragma unroll
      for (int j = 0; j < HP; ++j)
        if (j < hid) out[e * hid + j] = (y[j] - mean) * rstd * s_w[j] + s_b[j];
    }
  }
}

template <int CP, int HP>
int launch_mos(const float *ev, int64_t E, int cin, int hid, const int64_t *src, const int64_t *pos, int64_t R,
               int A, const float *ws, int As, const float *wq, const float *wv, const float *wg, const float *wo,
               const float *wgp, int Ag, const float *win, const float *ln_w, const float *ln_b, float eps,
               float *out, const MosWs &w, hipStream_t st) {
  typedef MosW<CP, HP> L;
  const bool fold = L::fold_bytes(As, Ag) <= kMaxLds;
  if (R > 0) {
    const int64_t n_win = (R + kWin - 1) / kWin;
    const int64_t wgs = std::min<int64_t>((n_win + 3) / 4, 2048);
    if (fold) {
      const int64_t nf = static_cast<int64_t>(L::fold_floats(As, Ag));
      hipLaunchKernelGGL((mos_fold_weights<CP, HP>), dim3(grid_for(nf)), dim3(kThreads), 0, st, ws, As, wq, wv, wg, wo,
                         wgp, Ag, cin, hid, w.wfold);
      hipLaunchKernelGGL((mos_patch_kernel<CP, HP, true>), dim3(static_cast<unsigned>(wgs)), dim3(kThreads),
                         L::fold_bytes(As, Ag), st, ev, E, cin, hid, src, pos, R, w.start, A, ws, As, wq, wv, wg, wo,
                         wgp, Ag, w.wfold, w.orow);
    } else {
      hipLaunchKernelGGL((mos_patch_kernel<CP, HP, false>), dim3(static_cast<unsigned>(wgs)), dim3(kThreads),
                         L::bytes(As, Ag), st, ev, E, cin, hid, src, pos, R, w.start, A, ws, As, wq, wv, wg, wo, wgp,
                         Ag, w.wfold, w.orow);
    }
  }
  if (E > 0)
    hipLaunchKernelGGL((mos_event_kernel<CP, HP>), dim3(grid_for(E)), dim3(kThreads), 0, st, ev, E, cin, hid, A,
                       w.dst, w.orow, R, win, ln_w, ln_b, eps, out);
  return launch_status("mos_attention_fwd");
}

// (cin, hid) -> the instantiated (CP, HP) that runs it ({0, 0}: not
// supported): the first template, in order of cost, that covers both sizes
// (the reference model's layers have exact ones).
struct Tpl {
  int cp, hp;
};
constexpr Tpl kTpls[] = {{2, 12}, {12, 12}, {16, 16}, {12, 24}, {24, 24}, {24, 32}, {32, 32}};
inline Tpl pick_tpl(int cin, int hid) {
  if (cin <= 0 || hid <= 0) return {0, 0};
  for (const Tpl &t : kTpls)
    if (cin <= t.cp && hid <= t.hp) return t;
  return {0, 0};
}

// LDS of the small kernels' weights: the folded weights when they fit,
// else the plain ones.
inline size_t small_lds(const Tpl &t, int A, int As, int Ag) {
  const size_t kS = t.hp * t.cp + 4, kG = t.hp * t.hp + 4;
  const size_t fold = sizeof(float) * (3 * As * kS + Ag * kG);
  const size_t plain = sizeof(float) * (As * kS + Ag * kG + 4 * static_cast<size_t>(t.hp) * t.hp);
  (void)A;
  return fold <= kMaxLds ? fold : plain;
}

}  // namespace

// The matrix-core path for sizes the small kernels do not take
// (mos_attention_mfma.hip).
namespace mosm {
bool supported(int cin, int H, int A);
size_t workspace_bytes(int64_t E, int cin, int H, int A, int64_t R, int64_t P);
size_t lds_bytes(int cin, int H);
int forward(const float *events, int64_t E, int cin, const int64_t *row_src, const int64_t *row_pos, int64_t R,
            const int64_t *patch_len, int64_t P, int A, const float *w_scatter, int As, const float *w_q,
            const float *w_v, const float *w_g, const float *w_o, const float *w_gather, int Ag, const float *w_in,
            const float *ln_w, const float *ln_b, float eps, int H, float *out, void *workspace,
            size_t workspace_bytes_given, hipStream_t st);
}  // namespace mosm

namespace {
// Which kernels take a layer: 1 the small kernels (input and hidden <= 32,
// weights within 64 KB of LDS), 2 the matrix-core path (input and hidden
// multiples of 4 up to 128), 0 none.
inline int pick_path(int cin, int hid, int A, int As, int Ag) {
  if (A <= 0 || A > kMaxPos) return 0;
  const Tpl t = pick_tpl(cin, hid);
  if (t.hp != 0 && small_lds(t, A, As, Ag) <= kMaxLds) return 1;
  return mosm::supported(cin, hid, A) ? 2 : 0;
}
}  // namespace
}  // namespace ssla

extern "C" size_t ssla_mos_attention_workspace_size(int64_t n_events, int c_in, int hidden, int A, int64_t n_rows,
                                                    int64_t n_patches) {
  using namespace ssla;
  if (n_events < 0 || A <= 0 || A > kMaxPos || n_rows < 0 || n_patches < 0) return 0;
  // the larger of the two paths' needs (which one runs depends on the
  // projections' sharing, not known here)
  size_t bytes = 0;
  const Tpl t = pick_tpl(c_in, hidden);
  if (t.hp != 0) bytes = mos_layout(nullptr, n_events, A, n_rows, n_patches, t.cp, t.hp).total;
  if (mosm::supported(c_in, hidden, A))
    bytes = std::max(bytes, mosm::workspace_bytes(n_events, c_in, hidden, A, n_rows, n_patches));
  return bytes;
}

extern "C" size_t ssla_mos_attention_lds_bytes(int c_in, int hidden, int A, int scatter_per_pos, int gather_per_pos) {
  using namespace ssla;
  const int As = scatter_per_pos ? A : 1, Ag = gather_per_pos ? A : 1;
  switch (pick_path(c_in, hidden, A, As, Ag)) {
    case 1: return small_lds(pick_tpl(c_in, hidden), A, As, Ag);
    case 2: return mosm::lds_bytes(c_in, hidden);
    default: return 0;   // 0: the fused kernels do not take this layer
  }
}

extern "C" int ssla_mos_attention_fwd(const float *events, int64_t n_events, int c_in, const int64_t *row_src,
                                      const int64_t *row_pos, int64_t n_rows, const int64_t *patch_len,
                                      int64_t n_patches, int A, const float *w_scatter, int scatter_per_pos,
                                      const float *w_q, const float *w_v, const float *w_g, const float *w_o,
                                      const float *w_gather, int gather_per_pos, const float *w_in,
                                      const float *ln_w, const float *ln_b, float eps, int hidden, float *out,
                                      void *workspace, size_t workspace_bytes, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_events >= 0 && n_rows >= 0 && n_patches >= 0 && c_in > 0 && hidden > 0 && A > 0,
                 "mos_attention_fwd: bad sizes E=%lld R=%lld P=%lld cin=%d hidden=%d A=%d", (long long)n_events,
                 (long long)n_rows, (long long)n_patches, c_in, hidden, A);
  const int As = scatter_per_pos ? A : 1, Ag = gather_per_pos ? A : 1;
  const int path = pick_path(c_in, hidden, A, As, Ag);
  if (path == 0) {
    set_error("mos_attention_fwd: needs at most %d kernel positions and either input and hidden sizes up to 32 "
              "with weights within %zu bytes of LDS, or sizes that are multiples of 4 up to 128 "
              "(cin=%d hidden=%d A=%d)", kMaxPos, kMaxLds, c_in, hidden, A);
    return SSLA_ERR_UNSUPPORTED;
  }
  if (!w_in && c_in != hidden) {
    set_error("mos_attention_fwd: input size %d differs from hidden %d but no input projection given", c_in, hidden);
    return SSLA_ERR_ARG;
  }
  SSLA_CHECK_ARG(n_rows < 0x7fffffff && n_events * A < (int64_t{1} << 40), "mos_attention_fwd: too many rows");
  if (n_events == 0) return SSLA_OK;
  SSLA_CHECK_ARG(events && out && w_scatter && w_q && w_v && w_g && w_o && w_gather && ln_w && ln_b,
                 "mos_attention_fwd: null pointer");
  SSLA_CHECK_ARG(n_rows == 0 || (row_src && row_pos && patch_len), "mos_attention_fwd: null row arrays");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (path == 2) {
    SSLA_CHECK_ARG(aligned(events, 16) && (!w_in || aligned(w_in, 16)),
                   "mos_attention_fwd: events and w_in must be 16-byte aligned");
    return mosm::forward(events, n_events, c_in, row_src, row_pos, n_rows, patch_len, n_patches, A, w_scatter, As,
                         w_q, w_v, w_g, w_o, w_gather, Ag, w_in, ln_w, ln_b, eps, hidden, out, workspace,
                         workspace_bytes, st);
  }
  const Tpl tpl = pick_tpl(c_in, hidden);
  const MosWs w = mos_layout(workspace, n_events, A, n_rows, n_patches, tpl.cp, tpl.hp);
  if (!workspace || workspace_bytes < w.total) {
    set_error("mos_attention_fwd: workspace of %zu bytes needed, %zu given", w.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  hipLaunchKernelGGL(mos_fill_i32, dim3(grid_for(n_events * A)), dim3(kThreads), 0, st, w.dst, n_events * A, -1);
  hipLaunchKernelGGL(mos_fill_i32, dim3(1), dim3(kThreads), 0, st, reinterpret_cast<int32_t *>(w.orow + n_rows * tpl.hp),
                     static_cast<int64_t>(tpl.hp), 0);   // the zero row
  if (n_rows > 0) {
    hipLaunchKernelGGL(mos_fill_u8, dim3(grid_for(n_rows)), dim3(kThreads), 0, st, w.start, n_rows);
    if (n_patches > 0) {
      size_t tb = w.tmp_bytes;
      const hipError_t e = rocprim::exclusive_scan(w.tmp, tb, patch_len, w.cu, static_cast<int64_t>(0),
                                                   static_cast<size_t>(n_patches), rocprim::plus<int64_t>(), st);
      if (e != hipSuccess) {
        set_error("mos_attention_fwd: prefix sum failed: %s", hipGetErrorString(e));
        return SSLA_ERR_LAUNCH;
      }
      hipLaunchKernelGGL(mos_mark_starts, dim3(grid_for(n_patches)), dim3(kThreads), 0, st, w.cu, n_patches, n_rows,
                         w.start);
    }
    hipLaunchKernelGGL(mos_dst_fill, dim3(grid_for(n_rows)), dim3(kThreads), 0, st, row_src, row_pos, n_rows,
                       n_events, A, w.dst);
  }
#define MOS_CASE(C, H)                                                                                          \
  if (tpl.cp == C && tpl.hp == H)                                                                               \
    return launch_mos<C, H>(events, n_events, c_in, hidden, row_src, row_pos, n_rows, A, w_scatter, As, w_q, w_v, \
                            w_g, w_o, w_gather, Ag, w_in, ln_w, ln_b, eps, out, w, st);
  MOS_CASE(2, 12) MOS_CASE(12, 12) MOS_CASE(16, 16) MOS_CASE(12, 24) MOS_CASE(24, 24) MOS_CASE(24, 32)
  MOS_CASE(32, 32)
#undef MOS_CASE
  set_error("mos_attention_fwd: no kernel for cin=%d hidden=%d", c_in, hidden);
  return SSLA_ERR_UNSUPPORTED;
}
