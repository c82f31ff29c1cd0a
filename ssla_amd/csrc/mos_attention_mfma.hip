// MosAttention forward for hidden sizes above 32 (MOS_S stages 3-4, MOS_B),
// on fp32 matrix cores.
//
// Same computation as the fused kernels of mos_attention.hip (reference
// layers/mos_attention.py:75-167: scatter projection, q/v/g, sigmoid, the
// scan over every patch, o_proj, gather projection, the sum over an event's
// copies, residual, LayerNorm), with the projections as GEMMs over the pixel
// events instead of one lane per patch row.  Row r of the patch layout is
// the copy of pixel event src[r] at kernel position pos[r]; dst[e A + a] is
// the inverse map (or -1).
// * fold_kernel: the per-position matrices, once per call,
//     Wa[a] = [Wq; Wv; Wg] Ws[a]  ([3H, Cin]),  Wb[a] = Wgp[a] Wo  ([H, H]).
// * mos_in_kernel: [E, Cin] x [Cin, A 3H] (one shared Wa when the scatter
//   projection is shared), each output element (e, a, n) written to row
//   dst[e A + a] as q, v or sigmoid(g).  The events are read in order; no
//   row sort or gather.
// * mos_scan_kernel: h = a h + v along each patch's rows (zero start), and
//   q h written over q.
// * mos_out_split_kernel: per event, y = sum over a of Wb[a] (q h)[dst[e A + a]]
//   (+ Win e, or + e), i.e. [E, A H (+ Cin)] x [A H (+ Cin), H] with the
//   rows gathered, then LayerNorm over the event's H outputs in the same
//   workgroup.
// Products are v_mfma_f32_16x16x4_f32 (fp32 operands, exact products, fp32
// sums); the summation order differs from the reference's row by row
// GEMMs and index_add_ by rounding only.  q / v / a (then q h) live in the
// workspace as [R, H] fp32.
#include <cstring>
#include <rocprim/rocprim.hpp>

#include "common.h"

namespace ssla {
namespace mosm {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 64;     // events per GEMM tile
constexpr int kCols = 64;     // output columns per tile of the input GEMM
constexpr int kKc = 16;       // reduction elements staged per step
constexpr int kPad = 4;       // LDS row padding (floats)
constexpr int kMaxPosM = 49;  // kernel positions

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
  float *wa, *wb;      // folded matrices
  float *q, *v, *a;    // [R, H] each; q h replaces q after the scan
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

Ws layout(void *base, int64_t E, int cin, int H, int A, int64_t R, int64_t P) {
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
  w.wa = reinterpret_cast<float *>(take(sizeof(float) * static_cast<size_t>(A) * 3 * H * cin));
  w.wb = reinterpret_cast<float *>(take(sizeof(float) * static_cast<size_t>(A) * H * H));
  float **rows[3] = {&w.q, &w.v, &w.a};
  for (float **r : rows) *r = reinterpret_cast<float *>(take(sizeof(float) * static_cast<size_t>(R) * H));
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
// Four independent partial sums, so a thread's loads are not one chain.
__global__ void fold_kernel(const float *__restrict__ ws, int As, const float *__restrict__ wq,
                            const float *__restrict__ wv, const float *__restrict__ wg, const float *__restrict__ wo,
                            const float *__restrict__ wgp, int Ag, int cin, int H, float *__restrict__ wa,
                            float *__restrict__ wb) {
  const int64_t na = static_cast<int64_t>(As) * 3 * H * cin, nb = static_cast<int64_t>(Ag) * H * H;
  MOSM_GRID_STRIDE(i, na + nb) {
    const float *w1, *w2;
    int64_t stride;
    // (na + nb < 2^31, checked by the host: 32-bit index arithmetic)
    const uint32_t i32 = static_cast<uint32_t>(i);
    if (i < na) {
      const uint32_t ucin = static_cast<uint32_t>(cin), row = i32 / ucin;
      const int c = static_cast<int>(i32 - row * ucin);
      const uint32_t a = row / static_cast<uint32_t>(3 * H);
      const int n = static_cast<int>(row - a * static_cast<uint32_t>(3 * H));
      w1 = (n < H ? wq : n < 2 * H ? wv : wg) + static_cast<int64_t>(n % H) * H;
      w2 = ws + static_cast<int64_t>(a) * H * cin + c;
      stride = cin;
    } else {
      const uint32_t k = i32 - static_cast<uint32_t>(na), uh = static_cast<uint32_t>(H), row = k / uh;
      const int c = static_cast<int>(k - row * uh);
      const uint32_t a = row / uh;
      const int n = static_cast<int>(row - a * uh);
      w1 = wgp + (static_cast<int64_t>(a) * H + n) * H;
      w2 = wo + c;
      stride = H;
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    int j = 0;
    for (; j + 4 <= H; j += 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] = fmaf(w1[j + u], w2[(j + u) * stride], acc[u]);
    }
    for (; j < H; ++j) acc[0] = fmaf(w1[j], w2[j * stride], acc[0]);
    const float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    if (i < na) wa[i] = s;
    else wb[i - na] = s;
  }
}

// v_mfma_f32_16x16x4_f32 operand layout: lane l holds A[l % 16][l / 16] and
// B[l / 16][l % 16]; the accumulator holds D[4 (l / 16) + i][l % 16].

// The input GEMM.  Workgroup: (tile of kTile events, kCols columns of the
// As x 3H outputs); the four wavefronts own 32 x 32 quarters (2 x 2 MFMA
// tiles).  Each step stages kKc input channels of the events and of the
// weight rows in LDS, one 16-byte piece per thread each.  Column n' of the
// outputs is position a = n' / 3H (0 when the projection is shared: then
// every copy of the event takes the same value) and channel n = n' % 3H:
// q (n < H), v, or sigmoid(g) (n >= 2H), written to row dst[e A + a].
__global__ __launch_bounds__(kThreads) void mos_in_kernel(
    const float *__restrict__ X, int64_t E, int cin, const float *__restrict__ W, int As, int H, int A,
    const int32_t *__restrict__ dst, float *__restrict__ oq, float *__restrict__ ov, float *__restrict__ oa) {
  __shared__ __align__(16) float xs[kTile][kKc + kPad];
  __shared__ __align__(16) float wsm[kCols][kKc + kPad];
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int N1 = 3 * H, N = As * N1;
  const int c0 = blockIdx.y * kCols;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int sr = tid >> 2, sk = 4 * (tid & 3);
  const int64_t xe = e0 + sr;
  const int wcol = c0 + sr;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const int rb = 32 * (wv & 1), cb = 32 * (wv >> 1);
  for (int k0 = 0; k0 < cin; k0 += kKc) {
    const int k = k0 + sk;
    f32x4 xv = {0.f, 0.f, 0.f, 0.f}, wvv = {0.f, 0.f, 0.f, 0.f};
    if (k < cin) {   // cin is a multiple of 4: a piece is all in or all out
      if (xe < E) xv = *reinterpret_cast<const f32x4 *>(X + xe * cin + k);
      if (wcol < N) wvv = *reinterpret_cast<const f32x4 *>(W + static_cast<int64_t>(wcol) * cin + k);
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
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = c0 + cb + 16 * j + (lane & 15);
    if (col >= N) continue;
    const int a = col / N1, n = col - a * N1;
    float *o = n < H ? oq : n < 2 * H ? ov : oa;
    const int ch = n < H ? n : n < 2 * H ? n - H : n - 2 * H;
    const bool sig = n >= 2 * H;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t ev = e0 + rb + 16 * i + 4 * (lane >> 4) + e;
        if (ev >= E) continue;
        float val = acc[i][j][e];
        if (sig) val = __builtin_amdgcn_rcpf(1.f + fast_exp2(-val * kLog2e));
        if (As > 1) {
          const int32_t r = dst[ev * A + a];
          if (r >= 0) o[static_cast<int64_t>(r) * H + ch] = val;
        } else {
          for (int p = 0; p < A; ++p) {
            const int32_t r = dst[ev * A + p];
            if (r >= 0) o[static_cast<int64_t>(r) * H + ch] = val;
          }
        }
      }
  }
}

// h = a h + v along the rows of each patch (zero start), then q <- q h.
// One wavefront per patch; lane l holds channels l and l + 64.  The loads of
// kU rows go out before their serial fma chain.
constexpr int kU = 4;
__global__ __launch_bounds__(kThreads) void mos_scan_kernel(const int64_t *__restrict__ cu, int64_t P, int64_t R,
                                                            int H, float *__restrict__ q, const float *__restrict__ v,
                                                            const float *__restrict__ a) {
  const int lane = threadIdx.x & 63;
  const int64_t p = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  if (p >= P) return;
  const int64_t bos = min(max(cu[p], int64_t{0}), R), eos = min(max(cu[p + 1], bos), R);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int c = lane + 64 * half;
    if (c >= H) break;
    float h = 0.f;
    int64_t t = bos;
    for (; t + kU <= eos; t += kU) {
      float vv[kU], aa[kU], qq[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t o = (t + u) * H + c;
        vv[u] = v[o];
        aa[u] = a[o];
        qq[u] = q[o];
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        h = fmaf(aa[u], h, vv[u]);
        q[(t + u) * H + c] = qq[u] * h;
      }
    }
    for (; t < eos; ++t) {
      const int64_t o = t * H + c;
      h = fmaf(a[o], h, v[o]);
      q[o] = q[o] * h;
    }
  }
}

// The output GEMM with the copy sum, residual and LayerNorm, 16 events per
// workgroup: the reduction (the H channels of row dst[e A + a] of q h
// against Wb[a] for every position a, then the event's Cin inputs against
// Win) runs in chunks of 16 channels dealt round-robin to the four
// wavefronts.  Each wavefront accumulates all NT column tiles of the 16
// events from operands loaded straight from global memory in the MFMA
// layout (lane group g holding channels 4 g .. 4 g + 3 of a chunk in both
// operands), the next chunk's loads in flight while the current one is
// multiplied: no per-chunk barrier.  (A ring of three chunks in flight was
// slower: 54.0 / 62.9 against 49.7 / 58.3 µs at hidden 48 / 96, fewer
// wavefronts per SIMD.)  The four partial sums meet in LDS,
// and wavefront w finishes events 4 w .. 4 w + 3 (sum, identity residual,
// LayerNorm over H, store).
template <int NT>
__global__ __launch_bounds__(kThreads) void mos_out_split_kernel(
    const float *__restrict__ qh, int64_t R, const float *__restrict__ X, int64_t E, int cin, int H, int A,
    const int32_t *__restrict__ dst, const float *__restrict__ Wb, int Ag, const float *__restrict__ win,
    const float *__restrict__ ln_w, const float *__restrict__ ln_b, float eps, float *__restrict__ out) {
  constexpr int HP = 16 * NT;
  __shared__ int32_t s_dst[16 * kMaxPosM];
  __shared__ __align__(16) float part[4][16][HP + 4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * 16;
  for (int i = tid; i < 16 * A; i += kThreads) {
    const int64_t e = e0 + i / A;
    const int32_t r = e < E ? dst[e0 * A + i] : -1;
    s_dst[i] = (r >= 0 && r < R) ? r : -1;
  }
  __syncthreads();
  const int ch_h = (H + 15) / 16, ch_in = win ? (cin + 15) / 16 : 0;
  const int n_ch = A * ch_h + ch_in;
  const int64_t ev = e0 + c16;   // this lane's event (row of the first operand)
  auto load = [&](int s, f32x4 &xa, f32x4 (&wb)[NT]) __attribute__((always_inline)) {
    const bool res = s >= A * ch_h;
    const int a = res ? 0 : s / ch_h;
    const int k = (res ? s - A * ch_h : s - a * ch_h) * 16 + 4 * g;
    const int kd = res ? cin : H;
    xa = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (k < kd) {   // H and cin are multiples of 4: a piece is all in or all out
      if (res) {
        if (ev < E) xa = *reinterpret_cast<const f32x4 *>(X + ev * cin + k);
      } else {
        const int32_t r = s_dst[c16 * A + a];
        if (r >= 0) xa = *reinterpret_cast<const f32x4 *>(qh + static_cast<int64_t>(r) * H + k);
      }
    }
    const float *Wk = res ? win : Wb + (Ag > 1 ? static_cast<int64_t>(a) * H * H : 0);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = 16 * j + c16;
      wb[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
      if (n < H && k < kd) wb[j] = *reinterpret_cast<const f32x4 *>(Wk + static_cast<int64_t>(n) * kd + k);
    }
  };
  f32x4 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  f32x4 xa = {0.f, 0.f, 0.f, 0.f}, wb[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) wb[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  if (wv < n_ch) load(wv, xa, wb);
  for (int s = wv; s < n_ch; s += 4) {
    const bool more = s + 4 < n_ch;
    f32x4 xn = {0.f, 0.f, 0.f, 0.f}, wn[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) wn[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (more) load(s + 4, xn, wn);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[jj], wb[j][jj], acc[j], 0, 0, 0);
    xa = xn;
#pragma unroll
    for (int j = 0; j < NT; ++j) wb[j] = wn[j];
  }
  // acc[j][i] is event 4 g + i, column 16 j + c16
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) part[wv][4 * g + i][16 * j + c16] = acc[j][i];
  __syncthreads();
  // LayerNorm over the columns < H of events 4 wv .. 4 wv + 3; lane l holds
  // columns l and l + 64: the mean, then the mean square deviation from it
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int er = 4 * wv + i;
    const int64_t e = e0 + er;
    float y[2];
    float s1 = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int col = lane + 64 * hh;
      y[hh] = 0.f;
      if (col < H) {
        y[hh] = (part[0][er][col] + part[1][er][col]) + (part[2][er][col] + part[3][er][col]);
        if (!win && e < E) y[hh] += X[e * cin + col];
        s1 += y[hh];
      }
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) s1 += __shfl_xor(s1, m);
    const float mean = s1 / static_cast<float>(H);
    float s2 = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int col = lane + 64 * hh;
      if (col < H) s2 += (y[hh] - mean) * (y[hh] - mean);
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) s2 += __shfl_xor(s2, m);
    const float rstd = 1.f / sqrtf(s2 / static_cast<float>(H) + eps);
    if (e < E) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int col = lane + 64 * hh;
        if (col < H) out[e * H + col] = (y[hh] - mean) * rstd * ln_w[col] + ln_b[col];
      }
    }
  }
}

}  // namespace

bool supported(int cin, int H, int A) {
  return cin > 0 && H > 0 && cin <= 128 && H <= 128 && cin % 4 == 0 && H % 4 == 0 && A > 0 && A <= kMaxPosM;
}

// LDS of the largest kernel (the output GEMM at the padded hidden size).
size_t lds_bytes(int cin, int H) {
  (void)cin;
  const size_t hp = (H + 15) / 16 * 16;
  const size_t in_k = sizeof(float) * (kTile + kCols) * (kKc + kPad);
  const size_t out_k = sizeof(int32_t) * 16 * kMaxPosM + sizeof(float) * 4 * 16 * (hp + 4);
  return std::max(in_k, out_k);
}

size_t workspace_bytes(int64_t E, int cin, int H, int A, int64_t R, int64_t P) {
  return layout(nullptr, E, cin, H, A, R, P).total;
}

int forward(const float *events, int64_t E, int cin, const int64_t *row_src, const int64_t *row_pos, int64_t R,
            const int64_t *patch_len, int64_t P, int A, const float *w_scatter, int As, const float *w_q,
            const float *w_v, const float *w_g, const float *w_o, const float *w_gather, int Ag, const float *w_in,
            const float *ln_w, const float *ln_b, float eps, int H, float *out, void *workspace,
            size_t workspace_bytes_given, hipStream_t st) {
  const Ws w = layout(workspace, E, cin, H, A, R, P);
  if (!workspace || workspace_bytes_given < w.total) {
    set_error("mos_attention_fwd: workspace of %zu bytes needed, %zu given", w.total, workspace_bytes_given);
    return SSLA_ERR_WORKSPACE;
  }
  if (E == 0) return SSLA_OK;
  const int64_t tiles = (E + kTile - 1) / kTile;
  if (tiles > 0x7fffffff) {
    set_error("mos_attention_fwd: too many events");
    return SSLA_ERR_UNSUPPORTED;
  }
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
  }
  const int64_t nf = static_cast<int64_t>(As) * 3 * H * cin + static_cast<int64_t>(Ag) * H * H;
  if (nf >= 0x7fffffff) {
    set_error("mos_attention_fwd: folded weights too large");
    return SSLA_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(fold_kernel, dim3(grid_for(nf)), dim3(kThreads), 0, st, w_scatter, As, w_q, w_v, w_g, w_o,
                     w_gather, Ag, cin, H, w.wa, w.wb);
  if (R > 0) {
    const int N = As * 3 * H;
    hipLaunchKernelGGL(mos_in_kernel, dim3(static_cast<unsigned>(tiles), (N + kCols - 1) / kCols), dim3(kThreads), 0,
                       st, events, E, cin, w.wa, As, H, A, w.dst, w.q, w.v, w.a);
    if (P > 0) {
      const int64_t blocks = (P + kThreads / 64 - 1) / (kThreads / 64);
      if (blocks > 0x7fffffff) {
        set_error("mos_attention_fwd: too many patches");
        return SSLA_ERR_UNSUPPORTED;
      }
      hipLaunchKernelGGL(mos_scan_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st, w.cu, P, R, H,
                         w.q, w.v, w.a);
    }
  }
  const int64_t tiles16 = (E + 15) / 16;
  if (tiles16 > 0x7fffffff) {
    set_error("mos_attention_fwd: too many events");
    return SSLA_ERR_UNSUPPORTED;
  }
  switch ((H + 15) / 16) {
#define MOSM_OUT(NTV)                                                                                              \
  case NTV:                                                                                                        \
    hipLaunchKernelGGL((mos_out_split_kernel<NTV>), dim3(static_cast<unsigned>(tiles16)), dim3(kThreads), 0, st,  \
                       w.q, R, events, E, cin, H, A, w.dst, w.wb, Ag, w_in, ln_w, ln_b, eps, out);                 \
    break;
    MOSM_OUT(1) MOSM_OUT(2) MOSM_OUT(3) MOSM_OUT(4) MOSM_OUT(5) MOSM_OUT(6) MOSM_OUT(7) MOSM_OUT(8)
#undef MOSM_OUT
    default:
      set_error("mos_attention_fwd: hidden %d above 128", H);
      return SSLA_ERR_UNSUPPORTED;
  }
  return launch_status("mos_attention_fwd");
}

}  // namespace mosm
}  // namespace ssla
