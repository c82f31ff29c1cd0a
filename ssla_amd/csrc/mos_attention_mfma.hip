// MosAttention forward for hidden sizes above 32 (MOS_S stages 3-4, MOS_B),
// on fp32 matrix cores.
//
// Same computation as the fused kernels of mos_attention.hip (reference
// layers/mos_attention.py:75-167: scatter projection, q/v/g, sigmoid, the
// scan over every patch, o_proj, gather projection, the sum over an event's
// copies, residual, LayerNorm), but the projections run as GEMMs over the
// patch rows bucketed by kernel position instead of one lane per row:
// * the per-position matrices are folded once per call:
//   Wa[a] = [Wq; Wv; Wg] Ws[a]  ([3H, Cin]) and Wb[a] = Wgp[a] Wo ([H, H]);
// * the rows are bucketed by position with a stable device radix sort (no
//   host synchronisation) and cut into tiles of 64 rows of one position;
// * mos_gemm_kernel runs each tile against its position's matrix with
//   v_mfma_f32_16x16x4_f32 (fp32 operands: exact products, fp32 sums), the
//   first time gathering the rows' events and splitting the result into q,
//   v and sigmoid(g), the second time taking q * h as its input;
// * the varlen diagonal scan h = a h + v runs per patch (diag_scan.hip);
// * mos_rows_event_kernel sums every event's copies in increasing patch
//   order (decreasing kernel position, the order index_add_ visits them),
//   adds the residual (or its input projection) and applies LayerNorm, one
//   wavefront per event.
// All values are fp32; the row buffers (q, v, a, h, z) live in the workspace.
#include <cstring>
#include <rocprim/rocprim.hpp>

#include "common.h"

namespace ssla {
namespace mosm {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 64;     // rows per GEMM tile
constexpr int kCols = 64;     // columns per GEMM tile
constexpr int kKc = 16;       // reduction elements staged per step
constexpr int kPad = 4;       // LDS row padding (floats)
constexpr int kMaxEventWgs = 2048;

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
inline unsigned grid_for(int64_t n) {
  return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((n + kThreads - 1) / kThreads, 1 << 20)));
}
#define MOSM_GRID_STRIDE(i, n)                                                                  \
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < (n);      \
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)

struct Ws {
  int64_t *cu;         // [P + 1] patch row offsets
  int32_t *dst;        // [E * A] row of (event, position), or -1
  uint64_t *keys;      // [R] sorted positions
  int32_t *perm;       // [R] original row of each sorted position
  int64_t *boff;       // [A + 1] first sorted row of each position
  int64_t *toff;       // [A + 1] first tile of each position
  float *wa, *wb;      // folded matrices
  float *q, *v, *a, *h, *z;   // [R, H] each
  void *sort_tmp;
  size_t sort_bytes;
  void *scan_tmp;
  size_t scan_bytes;
  size_t total;
};

size_t excl_scan_bytes(int64_t n) {
  size_t tb = 0;
  (void)rocprim::exclusive_scan(nullptr, tb, static_cast<int64_t *>(nullptr), static_cast<int64_t *>(nullptr),
                                static_cast<int64_t>(0), static_cast<size_t>(std::max<int64_t>(n, 1)),
                                rocprim::plus<int64_t>());
  return tb;
}

Ws layout(void *base, int64_t E, int cin, int H, int A, int As, int Ag, int64_t R, int64_t P) {
  char *b = static_cast<char *>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char *p = b ? b + off : nullptr;
    off = align256(off + std::max<size_t>(bytes, 1));
    return p;
  };
  Ws w;
  w.cu = reinterpret_cast<int64_t *>(take(sizeof(int64_t) * (P + 1)));
  w.dst = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * static_cast<size_t>(E) * A));
  w.keys = reinterpret_cast<uint64_t *>(take(sizeof(uint64_t) * R));
  w.perm = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * R));
  w.boff = reinterpret_cast<int64_t *>(take(sizeof(int64_t) * (A + 1)));
  w.toff = reinterpret_cast<int64_t *>(take(sizeof(int64_t) * (A + 1)));
  w.wa = reinterpret_cast<float *>(take(sizeof(float) * static_cast<size_t>(As) * 3 * H * cin));
  w.wb = reinterpret_cast<float *>(take(sizeof(float) * static_cast<size_t>(Ag) * H * H));
  float **rows[5] = {&w.q, &w.v, &w.a, &w.h, &w.z};
  for (float **r : rows) *r = reinterpret_cast<float *>(take(sizeof(float) * static_cast<size_t>(R) * H));
  w.sort_bytes = ssla_sort_pairs_workspace_size(R);
  w.sort_tmp = take(w.sort_bytes);
  w.scan_bytes = excl_scan_bytes(P);
  w.scan_tmp = take(w.scan_bytes);
  w.total = off;
  return w;
}

__global__ void fill_i32(int32_t *p, int64_t n, int32_t v) { MOSM_GRID_STRIDE(i, n) p[i] = v; }

// dst[e * A + pos] = r for every row (each (event, position) pair occurs at
// most once); cu[P] = R.
__global__ void dst_fill(const int64_t *__restrict__ src, const int64_t *__restrict__ pos, int64_t R, int64_t E,
                         int A, int32_t *__restrict__ dst, int64_t *__restrict__ cu, int64_t P) {
  if (blockIdx.x == 0 && threadIdx.x == 0) cu[P] = R;
  MOSM_GRID_STRIDE(r, R) {
    const int64_t s = src[r], a = pos[r];
    if (s >= 0 && s < E && a >= 0 && a < A) dst[s * A + a] = static_cast<int32_t>(r);
  }
}

// Wa[a][n][c] = sum_j Wqvg[n][j] Ws[a][j][c]  (Wqvg = [Wq; Wv; Wg], [3H, H])
// Wb[a][n][c] = sum_j Wgp[a][n][j] Wo[j][c]
__global__ void fold_kernel(const float *__restrict__ ws, int As, const float *__restrict__ wq,
                            const float *__restrict__ wv, const float *__restrict__ wg, const float *__restrict__ wo,
                            const float *__restrict__ wgp, int Ag, int cin, int H, float *__restrict__ wa,
                            float *__restrict__ wb) {
  const int64_t na = static_cast<int64_t>(As) * 3 * H * cin, nb = static_cast<int64_t>(Ag) * H * H;
  MOSM_GRID_STRIDE(i, na + nb) {
    float acc = 0.f;
    if (i < na) {
      const int c = static_cast<int>(i % cin);
      const int n = static_cast<int>((i / cin) % (3 * H));
      const int64_t a = i / (static_cast<int64_t>(cin) * 3 * H);
      const float *w1 = (n < H ? wq : n < 2 * H ? wv : wg) + static_cast<int64_t>(n % H) * H;
      const float *w2 = ws + a * H * cin + c;
      for (int j = 0; j < H; ++j) acc = fmaf(w1[j], w2[static_cast<int64_t>(j) * cin], acc);
      wa[i] = acc;
    } else {
      const int64_t k = i - na;
      const int c = static_cast<int>(k % H);
      const int n = static_cast<int>((k / H) % H);
      const int64_t a = k / (static_cast<int64_t>(H) * H);
      const float *w1 = wgp + (a * H + n) * H;
      for (int j = 0; j < H; ++j) acc = fmaf(w1[j], wo[static_cast<int64_t>(j) * H + c], acc);
      wb[k] = acc;
    }
  }
}

// boff[a] = first sorted row with position >= a (a = 0..A), toff[a] = tiles
// of the positions before a (kTile rows each); one workgroup.
__global__ void bucket_kernel(const uint64_t *__restrict__ keys, int64_t R, int A, int64_t *__restrict__ boff,
                              int64_t *__restrict__ toff) {
  __shared__ int64_t s_b[64];
  const int a = threadIdx.x;
  if (a <= A) {
    int64_t lo = 0, hi = R;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (keys[mid] < static_cast<uint64_t>(a)) lo = mid + 1;
      else hi = mid;
    }
    s_b[a] = lo;
    boff[a] = lo;
  }
  __syncthreads();
  if (a == 0) {
    int64_t t = 0;
    for (int p = 0; p < A; ++p) {
      toff[p] = t;
      t += (s_b[p + 1] - s_b[p] + kTile - 1) / kTile;
    }
    toff[A] = t;
  }
}

// The last index j in [0, n) with off[j] <= x (off non-decreasing).
__device__ __forceinline__ int last_le(const int64_t *off, int n, int64_t x) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (off[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

enum { kLoadGather = 0, kLoadQH = 1 };
enum { kEpiQVA = 0, kEpiOut = 1 };

// One workgroup per (tile of kTile sorted rows of one position, kCols
// output columns); the four wavefronts own 32 x 32 quarters (2 x 2 MFMA
// tiles of 16 x 16).  Each step stages kKc reduction elements of the rows
// and of the weight rows in LDS (one 16-byte piece per thread each).
// v_mfma_f32_16x16x4_f32 operand layout: lane l holds A[l % 16][l / 16] and
// B[l / 16][l % 16]; the accumulator holds D[4 (l / 16) + i][l % 16].
template <int LOAD, int EPI>
__global__ __launch_bounds__(kThreads) void mos_gemm_kernel(
    const float *__restrict__ X, const float *__restrict__ X2, const int64_t *__restrict__ src, int64_t n_x,
    const int32_t *__restrict__ perm, const int64_t *__restrict__ boff, const int64_t *__restrict__ toff, int A,
    const float *__restrict__ W, int per_pos, int N, int Kd, int H, float *__restrict__ o0,
    float *__restrict__ o1, float *__restrict__ o2) {
  __shared__ __align__(16) float xs[kTile][kKc + kPad];
  __shared__ __align__(16) float wsm[kCols][kKc + kPad];
  __shared__ int32_t s_orig[kTile];
  __shared__ int64_t s_row[kTile];
  const int64_t t = blockIdx.x;
  if (t >= toff[A]) return;   // past the actual tile count (uniform over the workgroup)
  const int a = last_le(toff, A + 1, t);
  const int64_t r0 = boff[a] + (t - toff[a]) * kTile;
  const int nr = static_cast<int>(min(static_cast<int64_t>(kTile), boff[a + 1] - r0));
  const int c0 = blockIdx.y * kCols;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tid < kTile) {
    const int32_t o = tid < nr ? perm[r0 + tid] : -1;
    s_orig[tid] = o;
    int64_t row = -1;
    if (o >= 0) row = LOAD == kLoadGather ? src[o] : o;
    if (LOAD == kLoadGather && (row < 0 || row >= n_x)) row = -1;
    s_row[tid] = row;
  }
  __syncthreads();
  const float *Wa = W + (per_pos ? static_cast<int64_t>(a) * N * Kd : 0);
  // staging: thread tid loads piece (row tid / 4, elements 4 (tid % 4) .. +3)
  const int sr = tid >> 2, sk = 4 * (tid & 3);
  const int64_t xrow = s_row[sr];
  const int wcol = c0 + sr;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const int rb = 32 * (wv & 1), cb = 32 * (wv >> 1);
  for (int k0 = 0; k0 < Kd; k0 += kKc) {
    const int k = k0 + sk;
    f32x4 xv = {0.f, 0.f, 0.f, 0.f}, wvv = {0.f, 0.f, 0.f, 0.f};
    if (k < Kd) {   // Kd is a multiple of 4: a piece is all in or all out
      if (xrow >= 0) {
        xv = *reinterpret_cast<const f32x4 *>(X + xrow * Kd + k);
        if (LOAD == kLoadQH) xv *= *reinterpret_cast<const f32x4 *>(X2 + xrow * Kd + k);
      }
      if (wcol < N) wvv = *reinterpret_cast<const f32x4 *>(Wa + static_cast<int64_t>(wcol) * Kd + k);
    }
    __syncthreads();   // the previous step's operand reads are done
    *reinterpret_cast<f32x4 *>(&xs[sr][sk]) = xv;
    *reinterpret_cast<f32x4 *>(&wsm[sr][sk]) = wvv;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kKc / 4; ++kk) {
      const int kl = 4 * kk + (lane >> 4);
      float av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) av[i] = xs[rb + 16 * i + (lane & 15)][kl];
#pragma unroll
      for (int j = 0; j < 2; ++j) bv[j] = wsm[cb + 16 * j + (lane & 15)][kl];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
  }
  // epilogue: element (row rb + 16 i + 4 (lane / 16) + e, column cb + 16 j + lane % 16)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = rb + 16 * i + 4 * (lane >> 4) + e;
      if (row >= nr) continue;
      const int64_t o = s_orig[row];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = c0 + cb + 16 * j + (lane & 15);
        if (col >= N) continue;
        const float val = acc[i][j][e];
        if (EPI == kEpiQVA) {
          if (col < H) o0[o * H + col] = val;
          else if (col < 2 * H) o1[o * H + col - H] = val;
          else o2[o * H + col - 2 * H] = __builtin_amdgcn_rcpf(1.f + fast_exp2(-val * kLog2e));   // sigmoid
        } else {
          o0[o * N + col] = val;
        }
      }
    }
}

// Pixel events, one wavefront each (grid-stride): y = the sum of the
// event's copies' rows z (decreasing kernel position), plus the residual
// (Win e, or e), then LayerNorm; lane l holds channels l and l + 64.  With an
// input projection its transpose is staged in LDS (WinT[c][j], H * cin
// floats), so the lanes of a wavefront read consecutive words.
__global__ __launch_bounds__(kThreads) void mos_rows_event_kernel(
    const float *__restrict__ ev, int64_t E, int cin, int H, int A, const int32_t *__restrict__ dst,
    const float *__restrict__ z, int64_t R, const float *__restrict__ win, const float *__restrict__ ln_w,
    const float *__restrict__ ln_b, float eps, float *__restrict__ out) {
  extern __shared__ float win_t[];
  if (win) {
    for (int i = threadIdx.x; i < H * cin; i += kThreads) {
      const int j = i / cin, c = i - j * cin;
      win_t[c * H + j] = win[i];
    }
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int j0 = lane, j1 = lane + 64;
  const bool ok0 = j0 < H, ok1 = j1 < H;
  const float lw0 = ok0 ? ln_w[j0] : 0.f, lb0 = ok0 ? ln_b[j0] : 0.f;
  const float lw1 = ok1 ? ln_w[j1] : 0.f, lb1 = ok1 ? ln_b[j1] : 0.f;
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * (kThreads / 64);
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6); e < E; e += n_waves) {
    float y0 = 0.f, y1 = 0.f;
    for (int pa = A - 1; pa >= 0; --pa) {
      const int32_t r = dst[e * A + pa];
      if (r >= 0 && r < R) {
        if (ok0) y0 += z[static_cast<int64_t>(r) * H + j0];
        if (ok1) y1 += z[static_cast<int64_t>(r) * H + j1];
      }
    }
    const float *x = ev + e * cin;
    if (win) {
      float r0 = 0.f, r1 = 0.f;
      for (int c = 0; c < cin; ++c) {
        const float xc = x[c];
        if (ok0) r0 = fmaf(win_t[c * H + j0], xc, r0);
        if (ok1) r1 = fmaf(win_t[c * H + j1], xc, r1);
      }
      y0 += r0;
      y1 += r1;
    } else {
      if (ok0) y0 += x[j0];
      if (ok1) y1 += x[j1];
    }
    float s = (ok0 ? y0 : 0.f) + (ok1 ? y1 : 0.f);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    const float mean = s / static_cast<float>(H);
    const float d0 = ok0 ? y0 - mean : 0.f, d1 = ok1 ? y1 - mean : 0.f;
    float v = d0 * d0 + d1 * d1;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    const float rstd = 1.f / sqrtf(v / static_cast<float>(H) + eps);
    if (ok0) out[e * H + j0] = d0 * rstd * lw0 + lb0;
    if (ok1) out[e * H + j1] = d1 * rstd * lw1 + lb1;
  }
}

}  // namespace

bool supported(int cin, int H, int A) {
  return cin > 0 && H > 0 && cin <= 128 && H <= 128 && cin % 4 == 0 && H % 4 == 0 && A > 0 && A <= 63;
}

// LDS of the largest kernel: the GEMM tiles, or the event kernel's
// transposed input projection (present when cin != H).
size_t lds_bytes(int cin, int H) {
  const size_t gemm = sizeof(float) * (kTile + kCols) * (kKc + kPad) + (sizeof(int32_t) + sizeof(int64_t)) * kTile;
  const size_t ev = cin != H ? sizeof(float) * cin * H : 0;
  return std::max(gemm, ev);
}

size_t workspace_bytes(int64_t E, int cin, int H, int A, int64_t R, int64_t P) {
  return layout(nullptr, E, cin, H, A, A, A, R, P).total;
}

int forward(const float *events, int64_t E, int cin, const int64_t *row_src, const int64_t *row_pos, int64_t R,
            const int64_t *patch_len, int64_t P, int A, const float *w_scatter, int As, const float *w_q,
            const float *w_v, const float *w_g, const float *w_o, const float *w_gather, int Ag, const float *w_in,
            const float *ln_w, const float *ln_b, float eps, int H, float *out, void *workspace,
            size_t workspace_bytes_given, hipStream_t st) {
  const Ws w = layout(workspace, E, cin, H, A, A, A, R, P);
  if (!workspace || workspace_bytes_given < w.total) {
    set_error("mos_attention_fwd: workspace of %zu bytes needed, %zu given", w.total, workspace_bytes_given);
    return SSLA_ERR_WORKSPACE;
  }
  if (E == 0) return SSLA_OK;
  hipLaunchKernelGGL(fill_i32, dim3(grid_for(E * A)), dim3(kThreads), 0, st, w.dst, E * A, -1);
  if (R > 0) {
    if (P > 0) {
      size_t tb = w.scan_bytes;
      const hipError_t e = rocprim::exclusive_scan(w.scan_tmp, tb, patch_len, w.cu, static_cast<int64_t>(0),
                                                   static_cast<size_t>(P), rocprim::plus<int64_t>(), st);
      if (e != hipSuccess) {
        set_error("mos_attention_fwd: prefix sum failed: %s", hipGetErrorString(e));
        return SSLA_ERR_LAUNCH;
      }
    }
    hipLaunchKernelGGL(dst_fill, dim3(grid_for(R)), dim3(kThreads), 0, st, row_src, row_pos, R, E, A, w.dst, w.cu, P);
    const int64_t nf = static_cast<int64_t>(As) * 3 * H * cin + static_cast<int64_t>(Ag) * H * H;
    hipLaunchKernelGGL(fold_kernel, dim3(grid_for(nf)), dim3(kThreads), 0, st, w_scatter, As, w_q, w_v, w_g, w_o,
                       w_gather, Ag, cin, H, w.wa, w.wb);
    // rows bucketed by position (stable), tiles of kTile rows per position
    int end_bit = 1;
    while ((1 << end_bit) < A) ++end_bit;
    int s = ssla_sort_pairs(reinterpret_cast<const uint64_t *>(row_pos), nullptr, R, end_bit, w.keys, w.perm,
                            w.sort_tmp, w.sort_bytes, st);
    if (s) return s;
    hipLaunchKernelGGL(bucket_kernel, dim3(1), dim3(64), 0, st, w.keys, R, A, w.boff, w.toff);
    const int64_t tiles_max = R / kTile + A + 1;
    if (tiles_max > 0x7fffffff) {
      set_error("mos_attention_fwd: too many rows");
      return SSLA_ERR_UNSUPPORTED;
    }
    // scatter projection folded with q / v / g: one bucket matrix per
    // position (or one matrix for all when the projection is shared)
    const int N1 = 3 * H;
    hipLaunchKernelGGL((mos_gemm_kernel<kLoadGather, kEpiQVA>),
                       dim3(static_cast<unsigned>(tiles_max), (N1 + kCols - 1) / kCols), dim3(kThreads), 0, st,
                       events, nullptr, row_src, E, w.perm, w.boff, w.toff, A, w.wa, As > 1 ? 1 : 0, N1, cin, H, w.q,
                       w.v, w.a);
    s = ssla_diag_scan_fwd(w.v, w.a, w.cu, static_cast<int>(P), R, H, w.h, st);
    if (s) return s;
    // o_proj folded with the gather projection, on q * h
    hipLaunchKernelGGL((mos_gemm_kernel<kLoadQH, kEpiOut>),
                       dim3(static_cast<unsigned>(tiles_max), (H + kCols - 1) / kCols), dim3(kThreads), 0, st, w.q,
                       w.h, nullptr, R, w.perm, w.boff, w.toff, A, w.wb, Ag > 1 ? 1 : 0, H, H, H, w.z, nullptr,
                       nullptr);
  }
  const int64_t blocks = std::min<int64_t>((E + kThreads / 64 - 1) / (kThreads / 64), kMaxEventWgs);
  const size_t lds = w_in ? sizeof(float) * H * cin : 0;
  hipLaunchKernelGGL(mos_rows_event_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), lds, st, events, E,
                     cin, H, A, w.dst, w.z, R, w_in, ln_w, ln_b, eps, out);
  return launch_status("mos_attention_fwd");
}

}  // namespace mosm
}  // namespace ssla
