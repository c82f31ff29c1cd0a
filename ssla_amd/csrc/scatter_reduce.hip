// Scatter-reduce along dim 0 with an index broadcast over channels:
// torch_scatter.scatter_max / scatter_mean as called by SparsePool.forward
// (reference layers/sparse_pooling.py:33; torch_scatter itself is an
// un-vendored dependency, so the semantics implemented are its documented
// ones: empty rows give 0 (max: argmax = E), mean = sum / max(count, 1)).
//
// Pipeline (all on the caller's stream, no host synchronisation, no memset):
//   unsorted index:  hist -> scan -> bucket -> reduce -> combine
//   sorted index:    bounds -> scan -> reduce -> combine
// * hist   : each workgroup counts the rows of a contiguous event range in an
//            LDS histogram (LDS-privatised atomics; no contended global
//            atomics) and writes it as one row of a [n_hist, n_out] matrix.
// * scan   : one thread per output row sums its matrix column (turning the
//            column into per-workgroup start offsets), then a single-pass
//            chained scan (decoupled look-back over dynamically numbered
//            workgroups) gives the row offsets `off` and the piece offsets
//            `poff`; it also writes the piece -> row table.
// * bucket : each workgroup re-reads its event range and places event ids
//            into the row-grouped permutation with LDS atomics on its own
//            start offsets.
// * bounds : (sorted index) off[r] = first e with index[e] >= r.
// * reduce : one wavefront per "piece" (at most kPiece events of one row);
//            lane = channel, so every row read is one coalesced 4*C-byte
//            load and each lane folds its channel in registers.  Rows of
//            one piece are finished in place; rows of several pieces leave
//            per-piece partials.
// * combine: one wavefront per row of several pieces folds the partials in
//            piece order.
// Max/argmax use an explicit (value, smallest index) comparison, so the
// result does not depend on the order in which events are visited: it is
// bit-exact and deterministic.  Mean sums in fp64 (partials folded in piece
// order) and rounds once.
#include "common.h"

namespace ssla {
namespace {

#ifndef SSLA_SR_EV_THREADS
#define SSLA_SR_EV_THREADS 1024
#endif
#ifndef SSLA_SR_MAX_HIST
#define SSLA_SR_MAX_HIST 64
#endif
#ifndef SSLA_SR_EV_PER_BLOCK
#define SSLA_SR_EV_PER_BLOCK 16384
#endif
#ifndef SSLA_SR_SCAN_CELLS
#define SSLA_SR_SCAN_CELLS 256
#endif
#ifndef SSLA_SR_LOADS
#define SSLA_SR_LOADS 8
#endif
#ifndef SSLA_SR_LDS_CELLS
#define SSLA_SR_LDS_CELLS 24576
#endif
constexpr int kPiece = 128;                          // events per wavefront piece (2 per lane)
constexpr int kLdsCells = SSLA_SR_LDS_CELLS;         // LDS histogram capacity (96 KB)
constexpr int kEvThreads = SSLA_SR_EV_THREADS;       // hist / bucket workgroup size
constexpr int kMaxHist = SSLA_SR_MAX_HIST;           // histogram rows (workgroups) at most
constexpr int kEvPerBlock = SSLA_SR_EV_PER_BLOCK;    // events per histogram workgroup (target)
constexpr int kScanCells = SSLA_SR_SCAN_CELLS;       // output rows per scan workgroup
constexpr int kScanTpc = 1024 / SSLA_SR_SCAN_CELLS;  // scan threads per output row

struct WsLayout {
  size_t status, errs, off, poff, desc, flags, hist, perm, part, total;
  int n_hist;
  int64_t max_pieces;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

inline int hist_rows(int64_t E, int64_t n_out) {
  if (n_out > kLdsCells) return 1;   // global-atomic counting (rows too many for LDS)
  const int64_t r = (E + kEvPerBlock - 1) / kEvPerBlock;
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kMaxHist, r)));
}

inline int64_t scan_blocks(int64_t n_out) { return (n_out + kScanCells - 1) / kScanCells; }

// Grid of the bounds kernel (sorted index); also the number of error slots.
inline int bounds_blocks(int64_t E) {
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(1024, (E + 1 + 255) / 256)));
}

inline WsLayout ws_layout(int64_t E, int C, int64_t n_out) {
  WsLayout L;
  L.n_hist = hist_rows(E, n_out);
  L.max_pieces = n_out + (E + kPiece - 1) / kPiece;
  const int n_err = std::max(L.n_hist, bounds_blocks(E));
  size_t p = 0;
  L.status = p; p += 256;   // [0] status word, [1] scan ticket
  L.errs = p;  p = align256(p + sizeof(int32_t) * n_err);
  L.off = p;   p = align256(p + sizeof(int32_t) * (n_out + 1));
  L.poff = p;  p = align256(p + sizeof(int32_t) * (n_out + 1));
  L.desc = p;  p = align256(p + sizeof(int4) * (L.max_pieces + 1));
  L.flags = p; p = align256(p + sizeof(uint64_t) * (scan_blocks(n_out) + 1));
  L.hist = p;  p = align256(p + sizeof(int32_t) * static_cast<size_t>(L.n_hist) * (n_out + 1));
  L.perm = p;  p = align256(p + sizeof(int32_t) * (E > 0 ? E : 1));
  L.part = p;  p = align256(p + static_cast<size_t>(L.max_pieces) * C * 8);
  L.total = p;
  return L;
}

__device__ __forceinline__ bool bad_row(int64_t r, int64_t n_out) { return r < 0 || r >= n_out; }

// Event range [e0, e1) of histogram row b (identical in hist and bucket).
__device__ __forceinline__ void event_range(int64_t E, int n_hist, int b, int64_t &e0, int64_t &e1) {
  const int64_t per = (E + n_hist - 1) / n_hist;
  e0 = min(E, per * b);
  e1 = min(E, e0 + per);
}

// Clears the scan ticket and look-back flags (kernel 1 of every pipeline).
__device__ __forceinline__ void clear_scan_state(int32_t *ticket, uint64_t *flags, int64_t n_flags) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *ticket = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_flags; i += stride)
    flags[i] = 0;
}

// ---------------------------------------------------------------- hist --
// LDS mode: row b of hist = counts of the events of range b.
// Global mode (n_out > kLdsCells): one shared row of global counters, which
// the preceding fill kernel cleared.
template <bool LDS>
__global__ __launch_bounds__(kEvThreads) void hist_kernel(
    const int64_t *__restrict__ index, int64_t E, int64_t n_out, int n_hist,
    int32_t *__restrict__ hist, int32_t *__restrict__ errs, int32_t *ticket, uint64_t *flags,
    int64_t n_flags) {
  clear_scan_state(ticket, flags, n_flags);
  bool bad = false;
  if constexpr (LDS) {
    __shared__ int32_t lh[kLdsCells];
#pragma unroll 8
    for (int64_t c = threadIdx.x; c < n_out; c += kEvThreads) lh[c] = 0;
    __syncthreads();
    int64_t e0, e1;
    event_range(E, n_hist, blockIdx.x, e0, e1);
    int64_t e = e0 + threadIdx.x;
    for (; e + 7 * kEvThreads < e1; e += 8 * kEvThreads) {
      int64_t r[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) r[u] = index[e + u * kEvThreads];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (bad_row(r[u], n_out)) bad = true;
        else atomicAdd(&lh[r[u]], 1);
      }
    }
    for (; e < e1; e += kEvThreads) {
      const int64_t r = index[e];
      if (bad_row(r, n_out)) bad = true;
      else atomicAdd(&lh[r], 1);
    }
    __syncthreads();
    int32_t *row = hist + static_cast<int64_t>(blockIdx.x) * (n_out + 1);
#pragma unroll 8
    for (int64_t c = threadIdx.x; c < n_out; c += kEvThreads) row[c] = lh[c];
  } else {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kEvThreads;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kEvThreads + threadIdx.x; e < E; e += stride) {
      const int64_t r = index[e];
      if (bad_row(r, n_out)) bad = true;
      else atomicAdd(&hist[r], 1);
    }
  }
  const int any_bad = __syncthreads_or(bad ? 1 : 0);
  if (threadIdx.x == 0) errs[blockIdx.x] = any_bad ? SSLA_ERR_ARG : SSLA_OK;
}

// -------------------------------------------------------------- bounds --
// Sorted index: start[r] = first e with index[e] >= r for r in [0, n_out],
// start[n_out] = E.  Every r is written by exactly one e when the index is
// sorted and in range; otherwise the error slot is set and the reduce
// kernel's clamps keep every access inside the tensors.
__global__ __launch_bounds__(256) void bounds_kernel(const int64_t *__restrict__ index, int64_t E,
                                                     int64_t n_out, int32_t *__restrict__ start,
                                                     int32_t *__restrict__ errs, int32_t *ticket,
                                                     uint64_t *flags, int64_t n_flags) {
  clear_scan_state(ticket, flags, n_flags);
  bool bad = false;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e <= E; e += stride) {
    int64_t prev = e > 0 ? index[e - 1] : -1;
    int64_t cur = e < E ? index[e] : n_out;
    if (e < E && bad_row(cur, n_out)) bad = true;
    if (cur < prev) bad = true;
    prev = max(min(prev, n_out), (int64_t)-1);
    cur = max(min(cur, n_out), (int64_t)-1);
    for (int64_t r = prev + 1; r <= cur; ++r) start[r] = static_cast<int32_t>(e);
  }
  const int any_bad = __syncthreads_or(bad ? 1 : 0);
  if (threadIdx.x == 0) errs[blockIdx.x] = any_bad ? SSLA_ERR_ARG : SSLA_OK;
}

// ---------------------------------------------------------------- scan --
// Look-back word: [63:62] state (0 none, 1 aggregate, 2 inclusive prefix),
// [61:31] event count, [30:0] piece count.
constexpr uint64_t kFlagAgg = 1ull << 62, kFlagIncl = 2ull << 62;
constexpr uint64_t kMask31 = 0x7fffffffull;

// Payloads saturate at 2^31 - 1, so inconsistent input (a broken "sorted"
// promise) can give wrong offsets but never touches the state bits, and the
// look-back always terminates.
__device__ __forceinline__ uint64_t pack_pair(int64_t cnt, int64_t pcs) {
  const uint64_t c = static_cast<uint64_t>(min(max(cnt, (int64_t)0), (int64_t)kMask31));
  const uint64_t p = static_cast<uint64_t>(min(max(pcs, (int64_t)0), (int64_t)kMask31));
  return (c << 31) | p;
}

__device__ __forceinline__ int64_t pieces_of(int64_t cnt) { return cnt > 0 ? (cnt + kPiece - 1) / kPiece : 1; }

// SORTED: counts are differences of `start` (the bounds kernel's output in
// hist row 0).  Otherwise: counts are column sums of the [n_hist, n_out]
// matrix, and each column is rewritten with its exclusive prefix (the start
// offset of each histogram workgroup inside the row).
template <bool SORTED>
__global__ __launch_bounds__(kScanCells *kScanTpc) void scan_kernel(
    int32_t *__restrict__ hist, int n_hist, int64_t n_out, int64_t E, int32_t *__restrict__ off,
    int32_t *__restrict__ poff, int4 *__restrict__ desc,
    int32_t *ticket, uint64_t *flags, const int32_t *__restrict__ errs, int n_err,
    int32_t *__restrict__ status, int64_t max_pieces) {
  __shared__ int s_bid;
  __shared__ int32_t s_part[kScanTpc][kScanCells];
  __shared__ int64_t s_cnt[kScanCells], s_pcs[kScanCells];
  __shared__ int64_t s_excl[2];
  const int tid = threadIdx.x;
  if (tid == 0) s_bid = atomicAdd(ticket, 1);
  __syncthreads();
  const int64_t bid = s_bid;
  const int lc = tid % kScanCells, grp = tid / kScanCells;
  const int64_t cell = bid * kScanCells + lc;
  const bool live = cell < n_out;

  int64_t cnt = 0;
  if (SORTED) {
    if (grp == 0 && live) {
      const int64_t a = min(max((int64_t)hist[cell], (int64_t)0), E);
      const int64_t b = min(max((int64_t)hist[cell + 1], (int64_t)0), E);
      cnt = max(b - a, (int64_t)0);
    }
  } else {
    // column segment [b0, b1) of this thread
    const int per = (n_hist + kScanTpc - 1) / kScanTpc;
    const int b0 = min(n_hist, grp * per), b1 = min(n_hist, b0 + per);
    int32_t v[(kMaxHist + kScanTpc - 1) / kScanTpc];
    int32_t sum = 0;
#pragma unroll
    for (int i = 0; i < (kMaxHist + kScanTpc - 1) / kScanTpc; ++i) {
      v[i] = (live && b0 + i < b1) ? hist[static_cast<int64_t>(b0 + i) * (n_out + 1) + cell] : 0;
    }
#pragma unroll
    for (int i = 0; i < (kMaxHist + kScanTpc - 1) / kScanTpc; ++i) sum += v[i];
    s_part[grp][lc] = sum;
    __syncthreads();
    int32_t run = 0;
    for (int g2 = 0; g2 < grp; ++g2) run += s_part[g2][lc];
#pragma unroll
    for (int i = 0; i < (kMaxHist + kScanTpc - 1) / kScanTpc; ++i) {
      if (live && b0 + i < b1) hist[static_cast<int64_t>(b0 + i) * (n_out + 1) + cell] = run;
      run += v[i];
    }
    if (grp == kScanTpc - 1) cnt = run;   // column total
  }
  const int owner = SORTED ? 0 : kScanTpc - 1;   // the thread that holds cnt
  if (grp == owner) {
    s_cnt[lc] = cnt;
    s_pcs[lc] = live ? pieces_of(cnt) : 0;
  }
  __syncthreads();
  // inclusive scan over the block's cells: wavefront scans, then carries
  __shared__ int64_t s_wc[kScanCells / 64], s_wp[kScanCells / 64];
  int64_t c = 0, p = 0;
  if (tid < kScanCells) {
    c = s_cnt[tid];
    p = s_pcs[tid];
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t c2 = __shfl_up(c, d), p2 = __shfl_up(p, d);
      if ((tid & 63) >= d) { c += c2; p += p2; }
    }
    if ((tid & 63) == 63) {
      s_wc[tid >> 6] = c;
      s_wp[tid >> 6] = p;
    }
  }
  __syncthreads();
  if (tid < kScanCells) {
    for (int q = 0; q < (tid >> 6); ++q) {
      c += s_wc[q];
      p += s_wp[q];
    }
    s_cnt[tid] = c;
    s_pcs[tid] = p;
  }
  __syncthreads();
  // Windowed look-back by the first wavefront: lane l reads the flag of
  // block bid-1-l; the walk stops at the nearest inclusive prefix.  The
  // payload travels inside the flag word, so relaxed agent-scope atomics
  // suffice (no fences, which would write back / invalidate the L2).
  if (tid < 64) {
    const int64_t agg_c = s_cnt[kScanCells - 1], agg_p = s_pcs[kScanCells - 1];
    int64_t ex_c = 0, ex_p = 0;
    if (bid > 0) {
      if (tid == 0)
        __hip_atomic_store(&flags[bid], kFlagAgg | pack_pair(agg_c, agg_p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      // Predecessors took their tickets before this block, so they are
      // resident and publish without waiting on later blocks: the spin ends.
      int64_t j_end = bid;   // blocks [0, j_end) not folded yet
      while (true) {
        const int64_t j = j_end - 1 - tid;
        const uint64_t w = j >= 0 ? __hip_atomic_load(&flags[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                  : kFlagIncl;   // before block 0: inclusive prefix 0
        const uint64_t st = w >> 62;
        const uint64_t incl = __builtin_amdgcn_ballot_w64(st == 2);
        const uint64_t none = __builtin_amdgcn_ballot_w64(st == 0);
        const int last = incl ? __builtin_ctzll(incl) : 63;   // lanes [0, last] are needed
        const uint64_t need = last == 63 ? ~0ull : ((2ull << last) - 1);
        if (none & need) {
          __builtin_amdgcn_s_sleep(1);
          continue;
        }
        int64_t vc = tid <= last ? static_cast<int64_t>((w >> 31) & kMask31) : 0;
        int64_t vp = tid <= last ? static_cast<int64_t>(w & kMask31) : 0;
        for (int d = 32; d >= 1; d >>= 1) {
          vc += __shfl_xor(vc, d);
          vp += __shfl_xor(vp, d);
        }
        ex_c += vc;
        ex_p += vp;
        if (incl) break;
        j_end -= 64;
      }
    } else {
      // error slots of the first kernel -> status word (the wavefront reads
      // them in parallel: block 0 gates every later block's look-back)
      int st = SSLA_OK;
      for (int i = tid; i < n_err; i += 64) {
        const int v = errs[i];
        if (v != SSLA_OK) st = v;
      }
      const uint64_t bad = __builtin_amdgcn_ballot_w64(st != SSLA_OK);
      if (bad) st = __shfl(st, static_cast<int>(__builtin_ctzll(bad)));
      if (tid == 0) *status = st;
    }
    if (tid == 0) {
      __hip_atomic_store(&flags[bid], kFlagIncl | pack_pair(ex_c + agg_c, ex_p + agg_p), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      s_excl[0] = ex_c;
      s_excl[1] = ex_p;
      if (bid == static_cast<int64_t>(gridDim.x) - 1) {
        off[n_out] = static_cast<int32_t>(ex_c + agg_c);
        poff[n_out] = static_cast<int32_t>(ex_p + agg_p);
      }
    }
  }
  __syncthreads();
  if (grp == 0 && live) {
    const int64_t incl_c = s_cnt[lc], incl_p = s_pcs[lc];
    const int64_t c0 = s_excl[0] + incl_c - (lc > 0 ? s_cnt[lc] - s_cnt[lc - 1] : s_cnt[0]);
    const int64_t my_p = lc > 0 ? s_pcs[lc] - s_pcs[lc - 1] : s_pcs[0];
    const int64_t p0 = s_excl[1] + incl_p - my_p;
    off[cell] = static_cast<int32_t>(c0);
    poff[cell] = static_cast<int32_t>(p0);
    const int64_t cnt_me = lc > 0 ? s_cnt[lc] - s_cnt[lc - 1] : s_cnt[0];
    for (int64_t p = 0; p < my_p && p0 + p < max_pieces; ++p) {
      const int64_t rest = cnt_me - p * kPiece;
      desc[p0 + p] = make_int4(static_cast<int32_t>(cell), static_cast<int32_t>(c0 + p * kPiece),
                               static_cast<int32_t>(min(max(rest, (int64_t)0), (int64_t)kPiece)),
                               static_cast<int32_t>(my_p));
    }
  }
}

// -------------------------------------------------------------- bucket --
// perm[off[r] + start of this workgroup in row r + rank] = e.
template <bool LDS>
__global__ __launch_bounds__(kEvThreads) void bucket_kernel(
    const int64_t *__restrict__ index, int64_t E, int64_t n_out, int n_hist,
    const int32_t *__restrict__ off, int32_t *__restrict__ hist, int32_t *__restrict__ perm) {
  if constexpr (LDS) {
    __shared__ int32_t lc[kLdsCells];
    const int32_t *row = hist + static_cast<int64_t>(blockIdx.x) * (n_out + 1);
#pragma unroll 8
    for (int64_t c = threadIdx.x; c < n_out; c += kEvThreads) lc[c] = off[c] + row[c];
    __syncthreads();
    int64_t e0, e1;
    event_range(E, n_hist, blockIdx.x, e0, e1);
    int64_t e = e0 + threadIdx.x;
    for (; e + 7 * kEvThreads < e1; e += 8 * kEvThreads) {
      int64_t r[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) r[u] = index[e + u * kEvThreads];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (bad_row(r[u], n_out)) continue;
        const int32_t pos = atomicAdd(&lc[r[u]], 1);
        if (pos >= 0 && pos < E) perm[pos] = static_cast<int32_t>(e + u * kEvThreads);
      }
    }
    for (; e < e1; e += kEvThreads) {
      const int64_t r = index[e];
      if (bad_row(r, n_out)) continue;
      const int32_t pos = atomicAdd(&lc[r], 1);
      if (pos >= 0 && pos < E) perm[pos] = static_cast<int32_t>(e);
    }
  } else {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kEvThreads;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kEvThreads + threadIdx.x; e < E; e += stride) {
      const int64_t r = index[e];
      if (bad_row(r, n_out)) continue;
      const int32_t pos = off[r] + atomicAdd(&hist[r], 1);
      if (pos >= 0 && pos < E) perm[pos] = static_cast<int32_t>(e);
    }
  }
}

// -------------------------------------------------------------- reduce --
__device__ __forceinline__ void max_update(float x, int32_t e, float &best, int32_t &bidx) {
  if (x > best || (x == best && e < bidx)) { best = x; bidx = e; }
}

// Lane layout: a row of C floats is read as C/VW vectors of VW floats; lpr
// lanes (a power of two, at most 64) cover one row, so one instruction reads
// rpi = 64/lpr rows and kLoads instructions keep kLoads*rpi rows in flight.
// Rows wider than 64 vectors are split into column blocks.  The row groups
// of a wavefront are folded with xor shuffles at the end.
template <int VW> struct VecT;
template <> struct VecT<1> { typedef float T; };
template <> struct VecT<4> { typedef float4 T; };

template <int VW>
__device__ __forceinline__ float comp(const typename VecT<VW>::T &x, int i) {
  if constexpr (VW == 1) return x;
  else return i == 0 ? x.x : i == 1 ? x.y : i == 2 ? x.z : x.w;
}

constexpr int kLoads = SSLA_SR_LOADS;   // load instructions in flight per wavefront

template <bool MEAN, bool PERM, int VW>
__global__ __launch_bounds__(256) void reduce_kernel(
    const float *__restrict__ src, const int32_t *__restrict__ perm, const int32_t *__restrict__ poff,
    const int4 *__restrict__ desc, int64_t n_out, int64_t E, int C, int64_t max_pieces,
    float *__restrict__ out, int64_t *__restrict__ argmax, float *__restrict__ part_v,
    int32_t *__restrict__ part_i, double *__restrict__ part_s) {
  typedef typename VecT<VW>::T Vec;
  const int lane = threadIdx.x & 63;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t n_pieces = min(max((int64_t)poff[n_out], (int64_t)0), max_pieces);
  if (w >= n_pieces) return;   // wavefront-uniform
  const int4 d = desc[w];
  const int64_t r = min(max((int64_t)d.x, (int64_t)0), n_out - 1);
  const int64_t s = min(max((int64_t)d.y, (int64_t)0), E);
  const int n = static_cast<int>(min(max((int64_t)d.z, (int64_t)0), min((int64_t)kPiece, E - s)));
  const bool single = d.w <= 1;

  // event ids of this piece: lane l holds entries l and 64 + l
  int32_t pe0 = 0, pe1 = 0;
  if (PERM) {
    if (lane < n) pe0 = perm[s + lane];
    if (64 + lane < n) pe1 = perm[s + 64 + lane];
  }
  const int32_t e_hi = static_cast<int32_t>(max(E - 1, (int64_t)0));
  const int cw = C / VW;                                   // vectors per row
  const int lpr = cw >= 64 ? 64 : (cw <= 1 ? 1 : 1 << (32 - __builtin_clz(cw - 1)));
  const int rpi = 64 / lpr;
  const int rg = lane / lpr, cl = lane % lpr;

  for (int cb = 0; cb < cw; cb += 64) {
    const int cv = cb + cl;
    const bool act = cl < min(64, cw - cb);
    float best[VW];
    int32_t bidx[VW];
    double sum[VW];
#pragma unroll
    for (int i = 0; i < VW; ++i) {
      best[i] = -INFINITY;
      bidx[i] = 0x7fffffff;
      sum[i] = 0.0;
    }
    for (int j = 0; j < n; j += kLoads * rpi) {
      int32_t ev[kLoads];
      Vec x[kLoads];
      bool ok[kLoads];
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int jj = j + u * rpi + rg;
        ok[u] = act && jj < n;
        int32_t e;
        if (PERM) {
          const int32_t a = __shfl(pe0, jj & 63), b = __shfl(pe1, jj & 63);
          e = min(max(jj < 64 ? a : b, 0), e_hi);
        } else {
          e = static_cast<int32_t>(min(s + jj, static_cast<int64_t>(e_hi)));
        }
        ev[u] = e;
        if (ok[u]) x[u] = *reinterpret_cast<const Vec *>(src + static_cast<int64_t>(e) * C + cv * VW);
      }
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        if (!ok[u]) continue;
#pragma unroll
        for (int i = 0; i < VW; ++i) {
          if (MEAN) sum[i] += static_cast<double>(comp<VW>(x[u], i));
          else max_update(comp<VW>(x[u], i), ev[u], best[i], bidx[i]);
        }
      }
    }
    // fold the rpi row groups (lanes cl, cl + lpr, ...)
    for (int m = lpr; m < 64; m <<= 1) {
#pragma unroll
      for (int i = 0; i < VW; ++i) {
        if (MEAN) {
          sum[i] += __shfl_xor(sum[i], m);
        } else {
          const float ov = __shfl_xor(best[i], m);
          const int32_t oi = __shfl_xor(bidx[i], m);
          max_update(ov, oi, best[i], bidx[i]);
        }
      }
    }
    if (!act || rg != 0) continue;
#pragma unroll
    for (int i = 0; i < VW; ++i) {
      const int64_t c = static_cast<int64_t>(cv) * VW + i;
      if (single) {
        const int64_t o = r * C + c;
        if (MEAN) {
          out[o] = n > 0 ? static_cast<float>(sum[i] / static_cast<double>(n)) : 0.f;
        } else if (bidx[i] == 0x7fffffff) {
          out[o] = 0.f;
          argmax[o] = E;
        } else {
          out[o] = best[i];
          argmax[o] = bidx[i];
        }
      } else {
        const int64_t o = w * C + c;
        if (MEAN) {
          part_s[o] = sum[i];
        } else {
          part_v[o] = best[i];
          part_i[o] = bidx[i];
        }
      }
    }
  }
}

// Rows with several pieces: fold the piece partials (one workgroup per
// output row; rows of one piece return at once).  Thread (q, c) folds the
// pieces p0 + q, p0 + q + 4, ... of channel c; the four subsets are then
// folded in order q = 0..3, so the result is the same on every run.
template <bool MEAN>
__global__ __launch_bounds__(256) void combine_kernel(
    const int32_t *__restrict__ off, const int32_t *__restrict__ poff, int64_t n_out, int64_t E, int C,
    int64_t max_pieces, float *__restrict__ out, int64_t *__restrict__ argmax,
    const float *__restrict__ part_v, const int32_t *__restrict__ part_i, const double *__restrict__ part_s) {
  __shared__ float s_v[4][64];
  __shared__ int32_t s_i[4][64];
  __shared__ double s_s[4][64];
  const int64_t r = blockIdx.x;
  const int64_t n_pieces = min(max((int64_t)poff[n_out], (int64_t)0), max_pieces);
  const int64_t p0 = min(max((int64_t)poff[r], (int64_t)0), n_pieces);
  const int64_t p1 = min(max((int64_t)poff[r + 1], p0), n_pieces);
  if (p1 - p0 <= 1) return;   // workgroup-uniform
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int64_t row_lo = min(max((int64_t)off[r], (int64_t)0), E);
  const int64_t cnt = min(max((int64_t)off[r + 1], row_lo), E) - row_lo;
  for (int cb = 0; cb < C; cb += 64) {
    const int c = cb + lane;
    float best = -INFINITY;
    int32_t bidx = 0x7fffffff;
    double sum = 0.0;
    if (c < C) {
      for (int64_t p = p0 + q; p < p1; p += 4 * 8) {
        float pv[8];
        int32_t pi[8];
        double ps[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int64_t pp = p + 4 * u;
          if (pp < p1) {
            const int64_t o = pp * C + c;
            if (MEAN) {
              ps[u] = part_s[o];
            } else {
              pv[u] = part_v[o];
              pi[u] = part_i[o];
            }
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (p + 4 * u < p1) {
            if (MEAN) sum += ps[u];
            else max_update(pv[u], pi[u], best, bidx);
          }
        }
      }
    }
    s_v[q][lane] = best;
    s_i[q][lane] = bidx;
    s_s[q][lane] = sum;
    __syncthreads();
    if (q == 0 && c < C) {
      for (int q2 = 1; q2 < 4; ++q2) {
        if (MEAN) sum += s_s[q2][lane];
        else max_update(s_v[q2][lane], s_i[q2][lane], best, bidx);
      }
      const int64_t o = r * C + c;
      if (MEAN) {
        out[o] = cnt > 0 ? static_cast<float>(sum / static_cast<double>(cnt)) : 0.f;
      } else if (bidx == 0x7fffffff) {
        out[o] = 0.f;
        argmax[o] = E;
      } else {
        out[o] = best;
        argmax[o] = bidx;
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void fill_i32(int32_t *__restrict__ p, int64_t n, int32_t val) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = val;
}

template <bool MEAN>
int run_scatter(const float *src, const int64_t *index, int64_t E, int C, int64_t n_out,
                int sorted, float *out, int64_t *argmax, void *ws, size_t ws_bytes, hipStream_t st) {
  const char *name = MEAN ? "scatter_mean" : "scatter_max";
  SSLA_CHECK_ARG(E >= 0 && n_out >= 0 && C > 0, "%s: bad sizes E=%lld C=%d n_out=%lld", name,
                 (long long)E, C, (long long)n_out);
  SSLA_CHECK_ARG(E < 0x7fffffff && n_out < (1 << 30), "%s: E must be < 2^31 and n_out < 2^30", name);
  const WsLayout L = ws_layout(E, C, n_out);
  if (ws == nullptr || ws_bytes < L.total) {
    set_error("%s: workspace of %zu bytes needed, %zu given", name, L.total, ws_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(aligned(ws, 16), "%s: workspace must be 16-byte aligned", name);
  char *base = static_cast<char *>(ws);
  int32_t *status = reinterpret_cast<int32_t *>(base + L.status);
  int32_t *ticket = status + 1;
  if (n_out == 0) {
    hipLaunchKernelGGL(fill_i32, dim3(1), dim3(64), 0, st, status, (int64_t)1, (int32_t)SSLA_OK);
    return launch_status(name);
  }
  SSLA_CHECK_ARG(out && (MEAN || argmax), "%s: null output pointer", name);
  SSLA_CHECK_ARG(E == 0 || (src && index), "%s: null input pointer", name);
  SSLA_CHECK_ARG(aligned(src, 4) && aligned(index, 8), "%s: misaligned src or index", name);
  int32_t *errs = reinterpret_cast<int32_t *>(base + L.errs);
  int32_t *off = reinterpret_cast<int32_t *>(base + L.off);
  int32_t *poff = reinterpret_cast<int32_t *>(base + L.poff);
  int4 *desc = reinterpret_cast<int4 *>(base + L.desc);
  uint64_t *flags = reinterpret_cast<uint64_t *>(base + L.flags);
  int32_t *hist = reinterpret_cast<int32_t *>(base + L.hist);
  int32_t *perm = reinterpret_cast<int32_t *>(base + L.perm);
  float *part_v = reinterpret_cast<float *>(base + L.part);
  int32_t *part_i = reinterpret_cast<int32_t *>(base + L.part + static_cast<size_t>(L.max_pieces) * C * 4);
  double *part_s = reinterpret_cast<double *>(base + L.part);
  const int64_t n_scan = scan_blocks(n_out);
  const bool lds = n_out <= kLdsCells;
  int n_err = 0;

  if (sorted) {
    const int nb = bounds_blocks(E);
    hipLaunchKernelGGL(bounds_kernel, dim3(nb), dim3(256), 0, st, index, E, n_out, hist, errs, ticket, flags,
                       n_scan + 1);
    n_err = nb;
    hipLaunchKernelGGL((scan_kernel<true>), dim3(static_cast<unsigned>(n_scan)), dim3(kScanCells * kScanTpc), 0,
                       st, hist, 1, n_out, E, off, poff, desc, ticket, flags, errs, n_err, status, L.max_pieces);
  } else {
    if (lds) {
      hipLaunchKernelGGL((hist_kernel<true>), dim3(L.n_hist), dim3(kEvThreads), 0, st, index, E, n_out,
                         L.n_hist, hist, errs, ticket, flags, n_scan + 1);
      n_err = L.n_hist;
    } else {
      hipLaunchKernelGGL(fill_i32, dim3(static_cast<unsigned>(std::min<int64_t>(1024, (n_out + 256) / 256))),
                         dim3(256), 0, st, hist, n_out + 1, 0);
      const int nb = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(1024, (E + kEvThreads - 1) / kEvThreads)));
      hipLaunchKernelGGL((hist_kernel<false>), dim3(nb), dim3(kEvThreads), 0, st, index, E, n_out, 1, hist, errs,
                         ticket, flags, n_scan + 1);
      n_err = nb;
    }
    hipLaunchKernelGGL((scan_kernel<false>), dim3(static_cast<unsigned>(n_scan)), dim3(kScanCells * kScanTpc), 0,
                       st, hist, L.n_hist, n_out, E, off, poff, desc, ticket, flags, errs, n_err, status, L.max_pieces);
    if (lds) {
      hipLaunchKernelGGL((bucket_kernel<true>), dim3(L.n_hist), dim3(kEvThreads), 0, st, index, E, n_out,
                         L.n_hist, off, hist, perm);
    } else {
      const int nb = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(1024, (E + kEvThreads - 1) / kEvThreads)));
      hipLaunchKernelGGL((bucket_kernel<false>), dim3(nb), dim3(kEvThreads), 0, st, index, E, n_out, 1, off, hist,
                         perm);
    }
  }
  const int64_t blocks = (L.max_pieces + 3) / 4;
  SSLA_CHECK_ARG(blocks <= 0x7fffffff, "%s: too many pieces", name);
  const bool vec4 = (C % 4) == 0 && aligned(src, 16);
  auto launch_reduce = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, src, perm, poff, desc, n_out,
                       E, C, L.max_pieces, out, argmax, part_v, part_i, part_s);
  };
  if (sorted) {
    if (vec4) launch_reduce(reduce_kernel<MEAN, false, 4>);
    else launch_reduce(reduce_kernel<MEAN, false, 1>);
  } else {
    if (vec4) launch_reduce(reduce_kernel<MEAN, true, 4>);
    else launch_reduce(reduce_kernel<MEAN, true, 1>);
  }
  hipLaunchKernelGGL((combine_kernel<MEAN>), dim3(static_cast<unsigned>(n_out)), dim3(256), 0, st, off,
                     poff, n_out, E, C, L.max_pieces, out, argmax, part_v, part_i, part_s);
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
