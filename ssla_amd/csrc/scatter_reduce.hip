// Scatter-reduce along dim 0 with an index broadcast over channels:
// torch_scatter.scatter_max / scatter_mean as called by SparsePool.forward
// (reference layers/sparse_pooling.py:33; torch_scatter itself is an
// un-vendored dependency, so the semantics implemented are its documented
// ones: empty rows give 0 (max: argmax = E), mean = sum / max(count, 1)).
//
// Pipeline (all on the caller's stream, no host synchronisation):
//   unsorted index:  zero -> count (int atomics) -> scan -> bucket -> reduce -> combine
//   sorted index:    zero -> boundaries (lower_bound per cell) -> scan -> reduce -> combine
// `bucket` writes a permutation that groups the events of each output row
// (a counting sort by row).  `reduce` gives one wavefront to each "piece"
// (up to kPiece consecutive events of one output row); rows that need a
// single piece are finished in place, longer rows leave per-piece partials
// that `combine` folds in piece order.  Max/argmax use an explicit
// (value, smallest index) comparison, so they do not depend on the order in
// which events are visited: the result is bit-exact and deterministic.
//
// Lane layout inside `reduce`: C/4 lanes read one 16-byte chunk each of an
// event row, so one wavefront instruction reads 64/(C/4) rows.
#include "common.h"

namespace ssla {
namespace {

constexpr int kPiece = 128;      // events per wavefront piece
constexpr int kScanThreads = 1024;

struct WsLayout {
  size_t status, off, poff, cur, perm, part, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

inline int64_t max_pieces(int64_t E, int64_t n_out) { return n_out + (E + kPiece - 1) / kPiece; }

inline WsLayout ws_layout(int64_t E, int C, int64_t n_out) {
  WsLayout L;
  size_t p = 0;
  L.status = p; p += 256;
  L.off = p;  p = align256(p + sizeof(int32_t) * (n_out + 1));
  L.poff = p; p = align256(p + sizeof(int32_t) * (n_out + 1));
  L.cur = p;  p = align256(p + sizeof(int32_t) * (n_out + 1));
  L.perm = p; p = align256(p + sizeof(int32_t) * (E > 0 ? E : 1));
  L.part = p; p = align256(p + static_cast<size_t>(max_pieces(E, n_out)) * C * 8);
  L.total = p;
  return L;
}

__global__ __launch_bounds__(256) void fill_i32(int32_t *__restrict__ p, int64_t n, int32_t val) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = val;
}

// count[index[e]] += 1
__global__ __launch_bounds__(256) void count_rows(const int64_t *__restrict__ index, int64_t E,
                                                  int64_t n_out, int32_t *__restrict__ cnt,
                                                  int32_t *__restrict__ status) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < E; e += stride) {
    const int64_t r = index[e];
    if (r < 0 || r >= n_out) { *status = SSLA_ERR_ARG; continue; }
    atomicAdd(&cnt[r], 1);
  }
}

// Sorted index: off[r] = first e with index[e] >= r, off[n_out] = E.
__global__ __launch_bounds__(256) void sorted_boundaries(const int64_t *__restrict__ index, int64_t E,
                                                         int64_t n_out, int32_t *__restrict__ off,
                                                         int32_t *__restrict__ status) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e <= E; e += stride) {
    int64_t prev = e > 0 ? index[e - 1] : -1;
    int64_t cur = e < E ? index[e] : n_out;
    if (e < E && (cur < 0 || cur >= n_out)) { *status = SSLA_ERR_ARG; }
    if (cur < prev) { *status = SSLA_ERR_ARG; }
    prev = max(min(prev, n_out), (int64_t)-1);
    cur = max(min(cur, n_out), (int64_t)-1);
    for (int64_t r = prev + 1; r <= cur; ++r) off[r] = static_cast<int32_t>(e);
  }
}

// One workgroup: exclusive scan of counts into off (unsorted) and of the
// per-row piece counts into poff; cur <- off for the bucketing pass.
template <bool FROM_COUNTS>
__global__ __launch_bounds__(kScanThreads) void scan_rows(int32_t *__restrict__ off,
                                                          int32_t *__restrict__ poff,
                                                          int32_t *__restrict__ cur, int64_t n_out,
                                                          int64_t E) {
  __shared__ int32_t s_cnt[kScanThreads];
  __shared__ int32_t s_pcs[kScanThreads];
  const int tid = threadIdx.x;
  const int64_t per = (n_out + kScanThreads - 1) / kScanThreads;
  const int64_t lo = min(n_out, per * tid), hi = min(n_out, lo + per);
  auto count_of = [&](int64_t r) -> int32_t {
    return FROM_COUNTS ? off[r] : off[r + 1] - off[r];
  };
  int32_t sc = 0, sp = 0;
  for (int64_t r = lo; r < hi; ++r) {
    const int32_t c = count_of(r);
    sc += c;
    sp += c > 0 ? (c + kPiece - 1) / kPiece : 1;
  }
  s_cnt[tid] = sc;
  s_pcs[tid] = sp;
  __syncthreads();
  for (int d = 1; d < kScanThreads; d <<= 1) {
    int32_t a = 0, b = 0;
    if (tid >= d) { a = s_cnt[tid - d]; b = s_pcs[tid - d]; }
    __syncthreads();
    s_cnt[tid] += a;
    s_pcs[tid] += b;
    __syncthreads();
  }
  int32_t rc = s_cnt[tid] - sc, rp = s_pcs[tid] - sp;  // exclusive prefixes
  // Each thread rewrites only off[lo, hi) (counts -> offsets); the sorted
  // path never writes off, so reading off[hi] of the next range is safe.
  for (int64_t r = lo; r < hi; ++r) {
    const int32_t c = count_of(r);
    if (FROM_COUNTS) {
      off[r] = rc;
      cur[r] = rc;
    }
    poff[r] = rp;
    rc += c;
    rp += c > 0 ? (c + kPiece - 1) / kPiece : 1;
  }
  if (tid == kScanThreads - 1) {
    if (FROM_COUNTS) off[n_out] = static_cast<int32_t>(E);
    poff[n_out] = s_pcs[kScanThreads - 1];
  }
}

// perm[cur[index[e]]++] = e
__global__ __launch_bounds__(256) void bucket_rows(const int64_t *__restrict__ index, int64_t E,
                                                   int64_t n_out, int32_t *__restrict__ cur,
                                                   int32_t *__restrict__ perm) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < E; e += stride) {
    const int64_t r = index[e];
    if (r < 0 || r >= n_out) continue;
    const int32_t pos = atomicAdd(&cur[r], 1);
    perm[pos] = static_cast<int32_t>(e);
  }
}

__device__ __forceinline__ void max_update(float x, int32_t e, float &best, int32_t &bidx) {
  if (x > best || (x == best && e < bidx)) { best = x; bidx = e; }
}

// Largest r in [0, n_out) with poff[r] <= w.
__device__ __forceinline__ int64_t find_row(const int32_t *__restrict__ poff, int64_t n_out, int64_t w) {
  int64_t lo = 0, hi = n_out - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (poff[mid] <= w) lo = mid; else hi = mid - 1;
  }
  return lo;
}

template <bool MEAN, bool PERM>
__global__ __launch_bounds__(256) void reduce_pieces(
    const float *__restrict__ src, const int32_t *__restrict__ perm,
    const int32_t *__restrict__ off, const int32_t *__restrict__ poff, int64_t n_out, int64_t E,
    int C, float *__restrict__ out, int64_t *__restrict__ argmax, float *__restrict__ part_v,
    int32_t *__restrict__ part_i) {
  __shared__ float s_v[4][64 * 4];
  __shared__ int32_t s_i[4][64 * 4];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + wv;
  if (w >= poff[n_out]) return;  // wavefront-uniform
  const int64_t r = find_row(poff, n_out, w);
  const int64_t piece = w - poff[r];
  const int64_t npieces = poff[r + 1] - poff[r];
  // Clamp so that inconsistent offsets (an index that broke the "sorted"
  // promise) can never address outside src / perm.
  const int64_t row_lo = min(max((int64_t)off[r], (int64_t)0), E);
  const int64_t row_hi = min(max((int64_t)off[r + 1], row_lo), E);
  const int64_t s = row_lo + piece * kPiece;
  const int64_t e_end = min(row_hi, s + kPiece);
  const int C4 = C >> 2;

  for (int cb = 0; cb < C4; cb += 64) {            // column blocks of 256 floats
    const int cw = min(64, C4 - cb);              // float4 columns in this block
    const int rpw = 64 / cw;                      // rows per wavefront instruction
    const int rg = lane / cw, c4 = cb + lane % cw;
    const bool active = rg < rpw;
    float b0 = -INFINITY, b1 = -INFINITY, b2 = -INFINITY, b3 = -INFINITY;
    int32_t i0 = 0x7fffffff, i1 = 0x7fffffff, i2 = 0x7fffffff, i3 = 0x7fffffff;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (active) {
      int64_t pos = s + rg;
      for (; pos + 3 * rpw < e_end; pos += 4 * rpw) {
        int32_t ev[4];
        float4 x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) ev[u] = PERM ? perm[pos + u * rpw] : static_cast<int32_t>(pos + u * rpw);
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = reinterpret_cast<const float4 *>(src + static_cast<int64_t>(ev[u]) * C)[c4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (MEAN) {
            a0 += x[u].x; a1 += x[u].y; a2 += x[u].z; a3 += x[u].w;
          } else {
            max_update(x[u].x, ev[u], b0, i0); max_update(x[u].y, ev[u], b1, i1);
            max_update(x[u].z, ev[u], b2, i2); max_update(x[u].w, ev[u], b3, i3);
          }
        }
      }
      for (; pos < e_end; pos += rpw) {
        const int32_t ev = PERM ? perm[pos] : static_cast<int32_t>(pos);
        const float4 x = reinterpret_cast<const float4 *>(src + static_cast<int64_t>(ev) * C)[c4];
        if (MEAN) {
          a0 += x.x; a1 += x.y; a2 += x.z; a3 += x.w;
        } else {
          max_update(x.x, ev, b0, i0); max_update(x.y, ev, b1, i1);
          max_update(x.z, ev, b2, i2); max_update(x.w, ev, b3, i3);
        }
      }
      // stage per-lane partials: slot (rg, column) in this wavefront's LDS area
      const int sl = (rg * cw + lane % cw) * 4;
      if (MEAN) {
        s_v[wv][sl + 0] = a0; s_v[wv][sl + 1] = a1; s_v[wv][sl + 2] = a2; s_v[wv][sl + 3] = a3;
      } else {
        s_v[wv][sl + 0] = b0; s_v[wv][sl + 1] = b1; s_v[wv][sl + 2] = b2; s_v[wv][sl + 3] = b3;
        s_i[wv][sl + 0] = i0; s_i[wv][sl + 1] = i1; s_i[wv][sl + 2] = i2; s_i[wv][sl + 3] = i3;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // fold the row groups in order; lane j < 4*cw owns float column cb*4 + j
    for (int j = lane; j < 4 * cw; j += 64) {
      const int col = j >> 2, comp = j & 3;
      float bv = MEAN ? 0.f : -INFINITY;
      int32_t bi = 0x7fffffff;
      for (int g2 = 0; g2 < rpw; ++g2) {
        const int sl = (g2 * cw + col) * 4 + comp;
        if (MEAN) bv += s_v[wv][sl];
        else max_update(s_v[wv][sl], s_i[wv][sl], bv, bi);
      }
      const int64_t c = static_cast<int64_t>(cb) * 4 + j;
      if (npieces == 1) {
        if (MEAN) {
          const int64_t cnt = row_hi - row_lo;
          out[r * C + c] = cnt > 0 ? bv / static_cast<float>(cnt) : 0.f;
        } else if (bi == 0x7fffffff) {
          out[r * C + c] = 0.f;
          argmax[r * C + c] = E;
        } else {
          out[r * C + c] = src[static_cast<int64_t>(bi) * C + c];
          argmax[r * C + c] = bi;
        }
      } else {
        part_v[w * C + c] = bv;
        if (!MEAN) part_i[w * C + c] = bi;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Rows with more than one piece: fold the piece partials in piece order.
template <bool MEAN>
__global__ __launch_bounds__(256) void combine_pieces(
    const float *__restrict__ src, const int32_t *__restrict__ off,
    const int32_t *__restrict__ poff, int64_t n_out, int64_t E, int C, int64_t n_pieces_max,
    float *__restrict__ out, int64_t *__restrict__ argmax, const float *__restrict__ part_v,
    const int32_t *__restrict__ part_i) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= n_out) return;
  const int64_t p0 = min(max((int64_t)poff[r], (int64_t)0), n_pieces_max);
  const int64_t p1 = min(max((int64_t)poff[r + 1], p0), n_pieces_max);
  if (p1 - p0 <= 1) return;
  const int lane = threadIdx.x & 63;
  const int64_t cnt = max((int64_t)off[r + 1] - (int64_t)off[r], (int64_t)1);
  for (int c = lane; c < C; c += 64) {
    float bv = MEAN ? 0.f : -INFINITY;
    int32_t bi = 0x7fffffff;
    for (int64_t p = p0; p < p1; ++p) {
      if (MEAN) bv += part_v[p * C + c];
      else max_update(part_v[p * C + c], part_i[p * C + c], bv, bi);
    }
    if (MEAN) {
      out[r * C + c] = bv / static_cast<float>(cnt);
    } else {
      const bool found = bi >= 0 && bi < E;
      out[r * C + c] = found ? src[static_cast<int64_t>(bi) * C + c] : 0.f;
      argmax[r * C + c] = found ? bi : E;
    }
  }
}

template <bool MEAN>
int run_scatter(const float *src, const int64_t *index, int64_t E, int C, int64_t n_out,
                int sorted, float *out, int64_t *argmax, void *ws, size_t ws_bytes, hipStream_t st) {
  const char *name = MEAN ? "scatter_mean" : "scatter_max";
  SSLA_CHECK_ARG(E >= 0 && n_out >= 0 && C > 0, "%s: bad sizes E=%lld C=%d n_out=%lld", name,
                 (long long)E, C, (long long)n_out);
  SSLA_CHECK_ARG(E < 0x7fffffff && n_out < 0x7fffffff, "%s: E and n_out must be < 2^31", name);
  if ((C & 3) != 0) {
    set_error("%s: C=%d must be a multiple of 4", name, C);
    return SSLA_ERR_UNSUPPORTED;
  }
  const WsLayout L = ws_layout(E, C, n_out);
  if (ws == nullptr || ws_bytes < L.total) {
    set_error("%s: workspace of %zu bytes needed, %zu given", name, L.total, ws_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(aligned(ws, 16), "%s: workspace must be 16-byte aligned", name);
  char *base = static_cast<char *>(ws);
  int32_t *status = reinterpret_cast<int32_t *>(base + L.status);
  hipLaunchKernelGGL(fill_i32, dim3(1), dim3(64), 0, st, status, (int64_t)64, 0);
  if (n_out == 0) return launch_status(name);
  SSLA_CHECK_ARG(out && (MEAN || argmax), "%s: null output pointer", name);
  SSLA_CHECK_ARG(E == 0 || (src && index), "%s: null input pointer", name);
  SSLA_CHECK_ARG(aligned(src, 16), "%s: src must be 16-byte aligned", name);
  int32_t *off = reinterpret_cast<int32_t *>(base + L.off);
  int32_t *poff = reinterpret_cast<int32_t *>(base + L.poff);
  int32_t *cur = reinterpret_cast<int32_t *>(base + L.cur);
  int32_t *perm = reinterpret_cast<int32_t *>(base + L.perm);
  float *part_v = reinterpret_cast<float *>(base + L.part);
  int32_t *part_i = reinterpret_cast<int32_t *>(base + L.part + static_cast<size_t>(max_pieces(E, n_out)) * C * 4);
  const int ev_blocks = static_cast<int>(std::min<int64_t>(4096, (E + 255) / 256 + 1));
  const bool use_perm = !sorted;
  hipLaunchKernelGGL(fill_i32, dim3(static_cast<unsigned>(std::min<int64_t>(1024, (n_out + 256) / 256))),
                     dim3(256), 0, st, off, n_out + 1, 0);
  if (use_perm) {
    hipLaunchKernelGGL(count_rows, dim3(ev_blocks), dim3(256), 0, st, index, E, n_out, off, status);
    hipLaunchKernelGGL(scan_rows<true>, dim3(1), dim3(kScanThreads), 0, st, off, poff, cur, n_out, E);
    hipLaunchKernelGGL(bucket_rows, dim3(ev_blocks), dim3(256), 0, st, index, E, n_out, cur, perm);
  } else {
    hipLaunchKernelGGL(sorted_boundaries, dim3(ev_blocks), dim3(256), 0, st, index, E, n_out, off, status);
    hipLaunchKernelGGL(scan_rows<false>, dim3(1), dim3(kScanThreads), 0, st, off, poff, cur, n_out, E);
  }
  const int64_t waves = max_pieces(E, n_out);
  const int64_t blocks = (waves + 3) / 4;
  SSLA_CHECK_ARG(blocks <= 0x7fffffff, "%s: too many pieces", name);
  if (use_perm)
    hipLaunchKernelGGL((reduce_pieces<MEAN, true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       src, perm, off, poff, n_out, E, C, out, argmax, part_v, part_i);
  else
    hipLaunchKernelGGL((reduce_pieces<MEAN, false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       src, perm, off, poff, n_out, E, C, out, argmax, part_v, part_i);
  hipLaunchKernelGGL((combine_pieces<MEAN>), dim3(static_cast<unsigned>((n_out + 3) / 4)), dim3(256), 0, st,
                     src, off, poff, n_out, E, C, waves, out, argmax, part_v, part_i);
  return launch_status(name);
}

}  // namespace
}  // namespace ssla

extern "C" size_t ssla_scatter_workspace_size(int64_t E, int C, int64_t n_out) {
  if (E < 0 || n_out < 0 || C <= 0) return 0;
  return ssla::ws_layout(E, C, n_out).total;
}

extern "C" int ssla_scatter_max(const float *src, const int64_t *index, int64_t E, int C,
                                int64_t n_out, int index_sorted, float *out, int64_t *argmax,
                                void *workspace, size_t workspace_bytes, void *stream) {
  ssla::clear_error();
  return ssla::run_scatter<false>(src, index, E, C, n_out, index_sorted, out, argmax, workspace,
                                  workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int ssla_scatter_mean(const float *src, const int64_t *index, int64_t E, int C,
                                 int64_t n_out, int index_sorted, float *out, void *workspace,
                                 size_t workspace_bytes, void *stream) {
  ssla::clear_error();
  return ssla::run_scatter<true>(src, index, E, C, n_out, index_sorted, out, nullptr, workspace,
                                 workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int ssla_scatter_check(const void *workspace, int *status_out, void *stream) {
  ssla::clear_error();
  SSLA_CHECK_ARG(workspace && status_out, "scatter_check: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t v = 0;
  hipError_t e = hipMemcpyAsync(&v, workspace, sizeof(int32_t), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    ssla::set_error("scatter_check: %s", hipGetErrorString(e));
    return SSLA_ERR_LAUNCH;
  }
  *status_out = v;
  return SSLA_OK;
}
