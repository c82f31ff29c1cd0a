// Scatter-reduce along dim 0 with an index broadcast over channels:
// torch_scatter.scatter_max / scatter_mean as called by SparsePool.forward
// (reference layers/sparse_pooling.py:33; torch_scatter itself is an
// un-vendored dependency, so the semantics implemented are its documented
// ones: empty rows give 0 (max: argmax = E), mean = sum / max(count, 1)).
//
// Pipeline (all on the caller's stream, no host synchronisation, no memset):
//   sorted index:    seg_reduce -> seg_fixup
//   unsorted index:  hist -> scan -> bucket -> seg_reduce -> seg_fixup
// * hist   : each workgroup counts the rows of a contiguous event range in an
//            LDS histogram (LDS-privatised atomics; no contended global
//            atomics) and writes it as one row of a [n_hist, n_out] matrix.
// * scan   : one thread per output row sums its matrix column (turning the
//            column into per-workgroup start offsets), then a single-pass
//            chained scan (decoupled look-back over dynamically numbered
//            workgroups) gives the row offsets `off`.
// * bucket : each workgroup re-reads its event range and places (event id,
//            row) pairs at their row-grouped positions with LDS atomics on
//            its own start offsets (one 8-byte store per event).
// * seg_reduce: one wavefront per tile of 64 consecutive positions (events
//            of a sorted index, or counting-sort positions) and block of 64
//            channels: the tile's rows are loaded into registers (lane =
//            channel, one coalesced row per load, all in flight at once),
//            then walked in order; rows inside the tile are written, rows
//            crossing the tile's edges leave pieces and a flag; empty rows
//            are written as such.  It also checks a sorted index for range
//            and order.
// * seg_fixup: one wavefront per 8 tiles loads their flags and pieces in one
//            batch, folds each crossing row's pieces in tile order and
//            writes the row.
// Max/argmax use an explicit (value, smallest event id) comparison (NaN
// never wins), so the result does not depend on the order in which events
// are visited: it is bit-exact and deterministic.  Mean sums in fp64 and
// rounds once (the unsorted path's fp64 sum order follows the LDS-atomic
// placement, so its last fp64 bits may vary between runs).
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
#ifndef SSLA_SR_LDS_CELLS
#define SSLA_SR_LDS_CELLS 24576
#endif
constexpr int kLdsCells = SSLA_SR_LDS_CELLS;         // LDS histogram capacity (96 KB)
constexpr int kEvThreads = SSLA_SR_EV_THREADS;       // hist / bucket workgroup size
constexpr int kMaxHist = SSLA_SR_MAX_HIST;           // histogram rows (workgroups) at most
constexpr int kEvPerBlock = SSLA_SR_EV_PER_BLOCK;    // events per histogram workgroup (target)
constexpr int kScanCells = SSLA_SR_SCAN_CELLS;       // output rows per scan workgroup
constexpr int kScanTpc = 1024 / SSLA_SR_SCAN_CELLS;  // scan threads per output row
#ifndef SSLA_SR_TILE
#define SSLA_SR_TILE 64
#endif
#ifndef SSLA_SR_SEG_WAVES
#define SSLA_SR_SEG_WAVES 4
#endif
constexpr int kTile = SSLA_SR_TILE;            // positions per tile (<= 64: one per lane)
constexpr int kSegWaves = SSLA_SR_SEG_WAVES;   // wavefronts (tiles) per workgroup

struct WsLayout {
  size_t status, errs, off, flags, hist, perm, seg_flags, pieces, total;
  int n_hist;
  int64_t n_tiles;   // tiles of kTile positions (for E positions)
  int64_t n_seg;     // (tile, channel block) pairs
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

inline int hist_rows(int64_t E, int64_t n_out) {
  if (n_out > kLdsCells) return 1;   // global-atomic counting (rows too many for LDS)
  const int64_t r = (E + kEvPerBlock - 1) / kEvPerBlock;
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kMaxHist, r)));
}

inline int64_t scan_blocks(int64_t n_out) { return (n_out + kScanCells - 1) / kScanCells; }

// Histogram workgroups of the global-counter mode (also their error slots).
inline int global_hist_blocks(int64_t E) {
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(1024, (E + kEvThreads - 1) / kEvThreads)));
}

inline WsLayout ws_layout(int64_t E, int C, int64_t n_out) {
  WsLayout L;
  L.n_hist = hist_rows(E, n_out);
  const int n_err = std::max(L.n_hist, global_hist_blocks(E));
  size_t p = 0;
  L.status = p; p += 256;   // [0] status word, [1] scan ticket
  L.errs = p;  p = align256(p + sizeof(int32_t) * n_err);
  L.off = p;   p = align256(p + sizeof(int32_t) * (n_out + 1));
  L.n_tiles = (E + kTile - 1) / kTile;
  L.n_seg = L.n_tiles * ((C + 63) / 64);
  L.flags = p; p = align256(p + sizeof(uint64_t) * (scan_blocks(n_out) + 1));
  L.hist = p;  p = align256(p + sizeof(int32_t) * static_cast<size_t>(L.n_hist) * (n_out + 1));
  L.perm = p;  p = align256(p + sizeof(int2) * (E > 0 ? E : 1));   // (event, row) per sorted position
  // per (tile, channel block): tail and head flags, and two pieces (tail,
  // head) of 64 packed 8-byte values each
  L.seg_flags = p; p = align256(p + sizeof(uint64_t) * 2 * static_cast<size_t>(L.n_seg));
  L.pieces = p; p = align256(p + static_cast<size_t>(L.n_seg) * 2 * 64 * 8);
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

// Clears the scan ticket and look-back flags (kernel 1 of the unsorted
// pipeline).
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
// ---------------------------------------------------------------- scan --
// Look-back word: [63:62] state (0 none, 1 aggregate, 2 inclusive prefix),
// [30:0] event count.  The count saturates at 2^31 - 1, so inconsistent
// input can give wrong offsets but never touches the state bits, and the
// look-back always terminates.
constexpr uint64_t kFlagAgg = 1ull << 62, kFlagIncl = 2ull << 62;
constexpr uint64_t kMask31 = 0x7fffffffull;

__device__ __forceinline__ uint64_t pack_count(int64_t cnt) {
  return static_cast<uint64_t>(min(max(cnt, (int64_t)0), (int64_t)kMask31));
}

// Counts are column sums of the [n_hist, n_out] histogram matrix; each
// column is rewritten with its exclusive prefix (the start offset of each
// histogram workgroup inside the row), and off = exclusive prefix of the
// counts over rows (off[n_out] = events kept).
__global__ __launch_bounds__(kScanCells *kScanTpc) void scan_kernel(
    int32_t *__restrict__ hist, int n_hist, int64_t n_out, int32_t *__restrict__ off, int32_t *ticket,
    uint64_t *flags, const int32_t *__restrict__ errs, int n_err, int32_t *__restrict__ status) {
  __shared__ int s_bid;
  __shared__ int32_t s_part[kScanTpc][kScanCells];
  __shared__ int64_t s_cnt[kScanCells];
  __shared__ int64_t s_wc[kScanCells / 64];
  __shared__ int64_t s_excl;
  const int tid = threadIdx.x;
  if (tid == 0) s_bid = atomicAdd(ticket, 1);
  __syncthreads();
  const int64_t bid = s_bid;
  const int lc = tid % kScanCells, grp = tid / kScanCells;
  const int64_t cell = bid * kScanCells + lc;
  const bool live = cell < n_out;

  // column segment [b0, b1) of this thread
  const int per = (n_hist + kScanTpc - 1) / kScanTpc;
  const int b0 = min(n_hist, grp * per), b1 = min(n_hist, b0 + per);
  int32_t v[(kMaxHist + kScanTpc - 1) / kScanTpc];
  int32_t sum = 0;
#pragma unroll
  for (int i = 0; i < (kMaxHist + kScanTpc - 1) / kScanTpc; ++i)
    v[i] = (live && b0 + i < b1) ? hist[static_cast<int64_t>(b0 + i) * (n_out + 1) + cell] : 0;
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
  if (grp == kScanTpc - 1) s_cnt[lc] = run;   // column total
  __syncthreads();
  // inclusive scan over the block's cells: wavefront scans, then carries
  int64_t c = 0;
  if (tid < kScanCells) {
    c = s_cnt[tid];
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t c2 = __shfl_up(c, d);
      if ((tid & 63) >= d) c += c2;
    }
    if ((tid & 63) == 63) s_wc[tid >> 6] = c;
  }
  __syncthreads();
  if (tid < kScanCells) {
    for (int q = 0; q < (tid >> 6); ++q) c += s_wc[q];
    s_cnt[tid] = c;
  }
  __syncthreads();
  // Windowed look-back by the first wavefront: lane l reads the flag of
  // block bid-1-l; the walk stops at the nearest inclusive prefix.  The
  // payload travels inside the flag word, so relaxed agent-scope atomics
  // suffice (no fences, which would write back / invalidate the L2).
  if (tid < 64) {
    const int64_t agg = s_cnt[kScanCells - 1];
    int64_t ex = 0;
    if (bid > 0) {
      if (tid == 0)
        __hip_atomic_store(&flags[bid], kFlagAgg | pack_count(agg), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
        int64_t vc = tid <= last ? static_cast<int64_t>(w & kMask31) : 0;
        for (int d = 32; d >= 1; d >>= 1) vc += __shfl_xor(vc, d);
        ex += vc;
        if (incl) break;
        j_end -= 64;
      }
    } else {
      // error slots of the first kernel -> status word (the wavefront reads
      // them in parallel: block 0 gates every later block's look-back)
      int st = SSLA_OK;
      for (int i = tid; i < n_err; i += 64) {
        const int e = errs[i];
        if (e != SSLA_OK) st = e;
      }
      const uint64_t bad = __builtin_amdgcn_ballot_w64(st != SSLA_OK);
      if (bad) st = __shfl(st, static_cast<int>(__builtin_ctzll(bad)));
      if (tid == 0) *status = st;
    }
    if (tid == 0) {
      __hip_atomic_store(&flags[bid], kFlagIncl | pack_count(ex + agg), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_excl = ex;
      if (bid == static_cast<int64_t>(gridDim.x) - 1) off[n_out] = static_cast<int32_t>(ex + agg);
    }
  }
  __syncthreads();
  if (grp == 0 && live) {
    const int64_t mine = lc > 0 ? s_cnt[lc] - s_cnt[lc - 1] : s_cnt[0];
    off[cell] = static_cast<int32_t>(s_excl + s_cnt[lc] - mine);
  }
}

// -------------------------------------------------------------- bucket --
// perm[off[r] + start of this workgroup in row r + rank] = (e, r): one
// 8-byte store per event (the positions are scattered, so each store is a
// partial line of its own).
template <bool LDS>
__global__ __launch_bounds__(kEvThreads) void bucket_kernel(
    const int64_t *__restrict__ index, int64_t E, int64_t n_out, int n_hist,
    const int32_t *__restrict__ off, int32_t *__restrict__ hist, int2 *__restrict__ perm) {
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
        if (pos >= 0 && pos < E) perm[pos] = make_int2(static_cast<int32_t>(e + u * kEvThreads), static_cast<int32_t>(r[u]));
      }
    }
    for (; e < e1; e += kEvThreads) {
      const int64_t r = index[e];
      if (bad_row(r, n_out)) continue;
      const int32_t pos = atomicAdd(&lc[r], 1);
      if (pos >= 0 && pos < E) perm[pos] = make_int2(static_cast<int32_t>(e), static_cast<int32_t>(r));
    }
  } else {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kEvThreads;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kEvThreads + threadIdx.x; e < E; e += stride) {
      const int64_t r = index[e];
      if (bad_row(r, n_out)) continue;
      const int32_t pos = off[r] + atomicAdd(&hist[r], 1);
      if (pos >= 0 && pos < E) perm[pos] = make_int2(static_cast<int32_t>(e), static_cast<int32_t>(r));
    }
  }
}

// ------------------------------------------------------------ segments --
// One wavefront per (tile of kTile consecutive positions, block of 64
// channels); positions are events of a sorted index, or counting-sort
// positions (rows non-decreasing either way).  Lane = channel: each position
// is one coalesced row load, and all kTile loads of the tile are in flight
// at once, into registers (no LDS: occupancy is bounded by registers only).
// The wavefront then walks the positions in order.  A row that begins and ends inside the tile is written directly.
// A row that crosses tile edges (tiles ts < ... < te) leaves one piece per
// tile: the "tail" piece of ts (the row leaves through its end), tail
// pieces of the "through" tiles between (each wholly that row) and the
// "head" piece of te (the row entered through its start).  Every tile
// writes its tail flag (state, row, event count, bad-index bit) whether or
// not it has a tail piece, so no clearing is needed; seg_fixup_kernel then
// folds each crossing row's pieces in tile order (deterministic) and writes
// it.  Rows without events between a tile's rows (and before the first /
// after the last row of the input) are written as empty rows.
// Tail flag: bits 62-63 state, bit 61 bad index seen, bits 31-60 row (n_out
// < 2^30), bits 0-30 events of the piece.  Head flag: events of the head
// piece.
constexpr uint64_t kSegThrough = 1ull << 62, kSegPiece = 2ull << 62, kSegBad = 1ull << 61;
__device__ __forceinline__ uint64_t seg_state(uint64_t f) { return f >> 62; }
__device__ __forceinline__ int32_t seg_row(uint64_t f) { return static_cast<int32_t>((f >> 31) & 0x3fffffffu); }
__device__ __forceinline__ int64_t seg_count(uint64_t f) { return static_cast<int64_t>(f & 0x7fffffffu); }

template <bool MEAN>
struct SegAcc;
template <> struct SegAcc<false> {
  float best;
  int32_t idx;   // -1: no event yet
  __device__ __forceinline__ void reset() { best = -INFINITY; idx = -1; }
  // (value, smallest event id) maximum, independent of visiting order; NaN
  // never wins (-1 as unsigned is above every event id).  Branch-free: two
  // compares and two selects per event.
  __device__ __forceinline__ void add(float x, int32_t e) {
    const bool take = (x > best) | ((x == best) & (static_cast<uint32_t>(e) < static_cast<uint32_t>(idx)));
    best = take ? x : best;
    idx = take ? e : idx;
  }
  __device__ __forceinline__ uint64_t pack() const {
    return (static_cast<uint64_t>(static_cast<uint32_t>(idx)) << 32) | __float_as_uint(best);
  }
  __device__ __forceinline__ void merge(uint64_t p) {
    const int32_t i = static_cast<int32_t>(p >> 32);
    if (i >= 0) add(__uint_as_float(static_cast<uint32_t>(p)), i);
  }
};
template <> struct SegAcc<true> {
  double sum;
  __device__ __forceinline__ void reset() { sum = 0.0; }
  __device__ __forceinline__ void add(float x, int32_t) { sum += static_cast<double>(x); }
  __device__ __forceinline__ uint64_t pack() const { return static_cast<uint64_t>(__double_as_longlong(sum)); }
  __device__ __forceinline__ void merge(uint64_t p) { sum += __longlong_as_double(static_cast<long long>(p)); }
};

// Final value of one output element.
template <bool MEAN>
__device__ __forceinline__ void seg_store(float *out, int64_t *argmax, int64_t o, const SegAcc<MEAN> &a, int64_t cnt,
                                          int64_t E) {
  if constexpr (MEAN) {
    out[o] = cnt > 0 ? static_cast<float>(a.sum / static_cast<double>(cnt)) : 0.f;
  } else {
    if (a.idx < 0) {
      out[o] = 0.f;
      argmax[o] = E;
    } else {
      out[o] = a.best;
      argmax[o] = a.idx;
    }
  }
}

template <bool MEAN>
__device__ __forceinline__ void seg_empty_rows(float *out, int64_t *argmax, int64_t r0, int64_t r1, int C, int col,
                                               bool act, int64_t E) {
  for (int64_t r = r0; r < r1; ++r) {
    if (act) {
      out[r * C + col] = 0.f;
      if constexpr (!MEAN) argmax[r * C + col] = E;
    }
  }
}

// PERM: positions are those of the counting sort (perm[p] = (event id,
// row), n_valid = positions kept); otherwise positions are events and
// rows come from the sorted index.  n_seg = (tile, block) pairs for E
// positions; flags [2][n_seg] (tail, head); pieces [2][n_seg][64].
template <bool MEAN, bool PERM>
__global__ __launch_bounds__(64 * kSegWaves) void seg_reduce_kernel(
    const float *__restrict__ src, const int64_t *__restrict__ index, const int2 *__restrict__ perm,
    const int32_t *__restrict__ n_valid, int64_t E, int C, int64_t n_out,
    float *__restrict__ out, int64_t *__restrict__ argmax, int64_t n_seg, uint64_t *__restrict__ flags,
    uint64_t *__restrict__ pieces, int32_t *__restrict__ status) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int ncb = (C + 63) / 64;
  const int64_t Ev = PERM ? min(max(static_cast<int64_t>(*n_valid), static_cast<int64_t>(0)), E) : E;
  const int64_t n_tiles = (Ev + kTile - 1) / kTile;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * kSegWaves + w;
  if (q == 0 && !PERM && lane == 0) *status = SSLA_OK;   // bad indices are raised by the fixup kernel
  if (n_tiles == 0) {   // no (valid) events: every row is empty
    if (q == 0)
      for (int cb = 0; cb < C; cb += 64) seg_empty_rows<MEAN>(out, argmax, 0, n_out, C, cb + lane, cb + lane < C, E);
    return;
  }
  const int64_t t = q / ncb;
  if (t >= n_tiles) return;   // wavefront-uniform
  const int cb = static_cast<int>(q - t * ncb);
  const int64_t seg = t * ncb + cb;   // this wavefront's flag / piece
  const int64_t e0 = t * kTile;
  const int ne = static_cast<int>(min(static_cast<int64_t>(kTile), Ev - e0));
  const int ne_u = __builtin_amdgcn_readfirstlane(ne);   // the same in every lane
  auto row_at = [&](int64_t p) -> int64_t { return PERM ? static_cast<int64_t>(perm[p].y) : index[p]; };
  auto clamp_row = [&](int64_t r) { return static_cast<int32_t>(min(max(r, static_cast<int64_t>(0)), n_out - 1)); };
  // row ids: one per lane, checked for range and order
  const int64_t prev = e0 > 0 ? row_at(e0 - 1) : -1;
  const int64_t next = e0 + ne < Ev ? row_at(e0 + ne) : n_out;
  const int64_t rr = lane < ne ? row_at(e0 + lane) : n_out;
  const int64_t rl = __shfl_up(rr, 1);
  const int64_t rbefore = lane == 0 ? max(prev, static_cast<int64_t>(-1)) : rl;
  const bool bad_l = lane < ne && (rr < 0 || rr >= n_out || rr < rbefore);
  const bool bad = !PERM && __builtin_amdgcn_ballot_w64(bad_l) != 0;
  // clamped (memory-safe) rows; with bad input the result is unspecified,
  // but the tile links below stay consistent, so every look-back ends
  const int32_t row = clamp_row(rr);
  // event id of each position (argmax value and source row)
  const int32_t ev = lane < ne ? (PERM ? min(max(perm[e0 + lane].x, 0), static_cast<int32_t>(E - 1))
                                       : static_cast<int32_t>(e0 + lane))
                               : (PERM ? 0 : static_cast<int32_t>(e0));
  const int32_t first = __builtin_amdgcn_readfirstlane(row);
  const int32_t last = __builtin_amdgcn_readlane(row, ne - 1);
  // tile t's first row continues tile t-1's last row exactly when tile t-1's
  // last row continues into tile t (the same clamped comparison)
  const bool open_start = e0 > 0 && clamp_row(prev) == first;
  const bool open_end = e0 + ne < Ev && clamp_row(next) == last;
  // positions (after the first) where the row changes; the shuffle runs
  // with every lane active (a lane masked off by a condition would read 0)
  const int32_t row_up = __shfl_up(row, 1);
  const uint64_t bnd = __builtin_amdgcn_ballot_w64(lane > 0 && lane < ne && row != row_up);
  const bool through = open_start && open_end && bnd == 0;   // the whole tile is one continuing row
  const int col = cb * 64 + lane;
  const bool act = col < C;

  // load the tile's rows of this channel block (positions past the tile
  // re-read its first event's row and are never used)
  const float *pc = src + min(col, C - 1);
  float xr[kTile];
#pragma unroll
  for (int e = 0; e < kTile; ++e) {
    const int32_t id = __builtin_amdgcn_readlane(ev, e < ne_u ? e : 0);
    xr[e] = pc[static_cast<int64_t>(id) * C];
  }
  // empty rows between the previous tile's last row and this tile's first
  if (!open_start) {
    const int64_t gap0 = e0 > 0 ? static_cast<int64_t>(clamp_row(prev)) + 1 : 0;
    seg_empty_rows<MEAN>(out, argmax, gap0, first, C, col, act, E);
  }
  SegAcc<MEAN> acc, head;   // head: the first row's piece when it began before the tile
  acc.reset();
  head.reset();
  int head_cnt = 0;
  bool in_head = open_start;   // the walk is still in that first row
  int32_t cur = first;
  int c0 = 0;   // first position of the current row inside the tile
  // a row that ends inside the tile: keep it as the head piece, or write it
  auto close_row = [&](int32_t r, int cnt) __attribute__((always_inline)) {
    if (in_head) {
      head = acc;
      head_cnt = cnt;
      in_head = false;
    } else if (act) {
      seg_store<MEAN>(out, argmax, static_cast<int64_t>(r) * C + col, acc, cnt, E);
    }
  };
  // event id of position e (a scalar): consecutive ids without a permutation
  auto ev_at = [&](int e) __attribute__((always_inline)) {
    return PERM ? __builtin_amdgcn_readlane(ev, e) : static_cast<int32_t>(e0) + e;
  };
  // eight positions per step (the loop is unrolled: registers are named
  // statically); a full step without a row boundary (the common case) runs
  // without any per-position test
#pragma unroll
  for (int e8 = 0; e8 < kTile; e8 += 8) {   // kTile is a multiple of 8
    if (e8 >= ne_u) break;
    float xv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) xv[k] = xr[e8 + k];
    const uint32_t bb = static_cast<uint32_t>(bnd >> e8) & 0xffu;   // boundaries in this step
    if (bb == 0 && e8 + 8 <= ne_u) {
#pragma unroll
      for (int k = 0; k < 8; ++k) acc.add(xv[k], ev_at(e8 + k));
      continue;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = e8 + k;
      if (e < ne_u) {
        if ((bb >> k) & 1) {   // wavefront-uniform: a new row starts at position e
          const int32_t r = __builtin_amdgcn_readlane(row, e);
          close_row(cur, e - c0);
          seg_empty_rows<MEAN>(out, argmax, static_cast<int64_t>(cur) + 1, r, C, col, act, E);
          cur = r;
          c0 = e;
          acc.reset();
        }
        acc.add(xv[k], ev_at(e));
      }
    }
  }
  // pieces of crossing rows and this tile's flags (plain stores: the fixup
  // kernel runs after this one)
  const bool head_open = open_start && !through;   // first row entered through the start, ends here
  uint64_t *tails = pieces, *heads = pieces + n_seg * 64;   // [n_seg][64] each
  uint64_t *tail_f = flags, *head_f = flags + n_seg;          // [n_seg] each
  uint64_t tf = (bad ? kSegBad : 0) | (static_cast<uint64_t>(last) << 31);
  if (open_end) {
    tails[seg * 64 + lane] = acc.pack();
    tf |= (through ? kSegThrough : kSegPiece) | static_cast<uint64_t>(ne_u - c0);
  } else {
    close_row(cur, ne_u - c0);
  }
  if (lane == 0) tail_f[seg] = tf;
  if (head_open) {
    heads[seg * 64 + lane] = head.pack();
    if (lane == 0) head_f[seg] = static_cast<uint64_t>(head_cnt);
  }
  if (t == n_tiles - 1) seg_empty_rows<MEAN>(out, argmax, static_cast<int64_t>(last) + 1, n_out, C, col, act, E);
}

// One wavefront per kFixTiles consecutive tiles (t0 ..) of one channel
// block.  One batch of loads brings everything the common case needs: lane
// l's tail flag of tile t0 + l (64 flags), the head flags of tiles t0 + 1 ..
// t0 + kFixTiles, and the tail pieces of tiles t0 .. and head pieces of
// tiles t0 + 1 .. (kFixTiles each, staged in LDS).  An owner is a tile whose
// tail piece starts a crossing row; a ballot over the through tiles gives
// the tile te where its row ends.  Each owner's row is folded in tile order
// from LDS and written; pieces beyond the staged ones (rows that run past
// the window) are loaded on the way.  Also raises the status word for bad
// indices.
#ifndef SSLA_SR_FIX_TILES
#define SSLA_SR_FIX_TILES 8
#endif
constexpr int kFixTiles = SSLA_SR_FIX_TILES;   // tiles per fixup wavefront (<= 64)
constexpr int kFixWaves = 4;
// 64-bit value of lane k (a scalar)
__device__ __forceinline__ uint64_t rl64(uint64_t v, int k) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int32_t>(v), k));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int32_t>(v >> 32), k));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
template <bool MEAN, bool PERM>
__global__ __launch_bounds__(64 * kFixWaves) void seg_fixup_kernel(int64_t E, const int32_t *__restrict__ n_valid,
                                                                   int C, float *__restrict__ out,
                                                                   int64_t *__restrict__ argmax, int64_t n_seg,
                                                                   const uint64_t *__restrict__ flags,
                                                                   const uint64_t *__restrict__ pieces,
                                                                   int32_t *__restrict__ status) {
  __shared__ uint64_t st_tail[kFixWaves][kFixTiles][64], st_head[kFixWaves][kFixTiles][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int ncb = (C + 63) / 64;
  const int64_t Ev = PERM ? min(max(static_cast<int64_t>(*n_valid), static_cast<int64_t>(0)), E) : E;
  const int64_t n_tiles = (Ev + kTile - 1) / kTile;
  const int64_t n_win = (n_tiles + kFixTiles - 1) / kFixTiles;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * kFixWaves + w;
  const int64_t win = q / ncb;
  if (win >= n_win) return;   // wavefront-uniform
  const int cb = static_cast<int>(q - win * ncb);
  const int64_t t0 = win * kFixTiles;
  const uint64_t *tails = pieces, *heads = pieces + n_seg * 64;
  const uint64_t *tail_f = flags, *head_f = flags + n_seg;
  auto piece = [&](const uint64_t *base, int64_t tile) { return base + (tile * ncb + cb) * 64 + lane; };
  // the batch (positions past the last tile re-read the last tile, unused)
  const int64_t j = t0 + lane;
  const uint64_t f = j < n_tiles ? tail_f[j * ncb + cb] : 0;
  uint64_t hf = 0;
  if constexpr (MEAN) hf = lane < kFixTiles && j + 1 < n_tiles ? head_f[(j + 1) * ncb + cb] : 0;
  uint64_t pt[kFixTiles], ph[kFixTiles];
#pragma unroll
  for (int k = 0; k < kFixTiles; ++k) {
    pt[k] = *piece(tails, min(t0 + k, n_tiles - 1));
    ph[k] = *piece(heads, min(t0 + 1 + k, n_tiles - 1));
  }
  if (!PERM && __builtin_amdgcn_ballot_w64(lane < kFixTiles && (f & kSegBad)) != 0 && lane == 0)
    *status = SSLA_ERR_ARG;
  const uint64_t thr = __builtin_amdgcn_ballot_w64(seg_state(f) == 1);
  uint32_t own =
      static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(lane < kFixTiles && j < n_tiles && seg_state(f) == 2));
  if (own == 0) return;
#pragma unroll
  for (int k = 0; k < kFixTiles; ++k) {
    st_tail[w][k][lane] = pt[k];
    st_head[w][k][lane] = ph[k];
  }
  __builtin_amdgcn_wave_barrier();
  // te of the owner in lane l: the first tile after it that is not through
  // (-1: the through tiles run past the 64 flags)
  const uint64_t rest = lane < 63 ? (~thr >> (lane + 1)) : 0;
  const int64_t te_l = rest ? j + 1 + static_cast<int64_t>(__builtin_ctzll(rest)) : -1;
  const int col = cb * 64 + lane;
  const bool act = col < C;
  const int64_t staged_end = t0 + kFixTiles;   // tails staged for tiles < staged_end, heads for tiles <= staged_end
  while (own) {   // wavefront-uniform
    const int k = __builtin_ctz(own);
    own &= own - 1;
    const int64_t ts = t0 + k;
    int64_t te = static_cast<int64_t>(rl64(te_l, k));
    if (te < 0) {   // through tiles run past the 64 flags: walk on
      for (int64_t w0 = t0 + 64;; w0 += 64) {
        const int64_t jj = w0 + lane;
        const uint64_t ff = jj < n_tiles ? tail_f[jj * ncb + cb] : 0;
        const uint64_t stop = __builtin_amdgcn_ballot_w64(seg_state(ff) != 1);
        if (stop) {
          te = w0 + static_cast<int64_t>(__builtin_ctzll(stop));
          break;
        }
      }
    }
    te = min(te, n_tiles - 1);   // (bad input only)
    SegAcc<MEAN> a;
    a.reset();
    // tail piece of ts, then the through tiles ts+1 .. te-1: staged ones from
    // LDS, later ones sixteen loads at a time
    a.merge(st_tail[w][k][lane]);
    const int64_t m_end = min(te, staged_end);
    for (int64_t m = ts + 1; m < m_end; ++m) a.merge(st_tail[w][m - t0][lane]);
    for (int64_t k0 = m_end > ts + 1 ? m_end : ts + 1; k0 < te; k0 += 16) {
      uint64_t pv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) pv[i] = *piece(tails, min(k0 + i, te - 1));
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (k0 + i < te) a.merge(pv[i]);
    }
    // head piece of te
    if (te > ts) a.merge(te <= staged_end ? st_head[w][te - t0 - 1][lane] : *piece(heads, te));
    int64_t cnt = 0;
    if constexpr (MEAN) {
      // tail piece + through tiles (kTile events each) + head piece
      const int64_t hck = te <= staged_end ? static_cast<int64_t>(rl64(hf, static_cast<int>(te - t0 - 1)))
                                           : static_cast<int64_t>(head_f[te * ncb + cb]);
      cnt = seg_count(rl64(f, k)) + (te - ts - 1) * kTile + (te > ts ? hck : 0);
    }
    const int32_t R = seg_row(rl64(f, k));
    if (act) seg_store<MEAN>(out, argmax, static_cast<int64_t>(R) * C + col, a, cnt, E);
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
  uint64_t *flags = reinterpret_cast<uint64_t *>(base + L.flags);
  int32_t *hist = reinterpret_cast<int32_t *>(base + L.hist);
  int2 *perm = reinterpret_cast<int2 *>(base + L.perm);
  const int64_t n_scan = scan_blocks(n_out);
  const bool lds = n_out <= kLdsCells;
  int n_err = 0;

  uint64_t *pieces = reinterpret_cast<uint64_t *>(base + L.pieces);
  const int64_t g = std::max<int64_t>(1, (L.n_seg + kSegWaves - 1) / kSegWaves);
  SSLA_CHECK_ARG(L.n_tiles < (1 << 29) && g < 0x7fffffff, "%s: too many events x channel blocks", name);
  uint64_t *seg_flags = reinterpret_cast<uint64_t *>(base + L.seg_flags);
  const int64_t gf =
      std::max<int64_t>(1, ((L.n_tiles + kFixTiles - 1) / kFixTiles * ((C + 63) / 64) + kFixWaves - 1) / kFixWaves);
  auto segments = [&](auto red, auto fix, const int2 *perm_p, const int32_t *n_valid) {
    hipLaunchKernelGGL(red, dim3(static_cast<unsigned>(g)), dim3(64 * kSegWaves), 0, st, src, index, perm_p,
                       n_valid, E, C, n_out, out, argmax, L.n_seg, seg_flags, pieces, status);
    hipLaunchKernelGGL(fix, dim3(static_cast<unsigned>(gf)), dim3(64 * kFixWaves), 0, st, E, n_valid, C, out, argmax, L.n_seg,
                       seg_flags, pieces, status);
  };
  if (sorted) {
    segments(seg_reduce_kernel<MEAN, false>, seg_fixup_kernel<MEAN, false>, nullptr, nullptr);
    return launch_status(name);
  }
  // unsorted: counting sort of the events by row, then the same segments
  // over the sorted positions
  if (lds) {
    hipLaunchKernelGGL((hist_kernel<true>), dim3(L.n_hist), dim3(kEvThreads), 0, st, index, E, n_out, L.n_hist,
                       hist, errs, ticket, flags, n_scan + 1);
    n_err = L.n_hist;
  } else {
    hipLaunchKernelGGL(fill_i32, dim3(static_cast<unsigned>(std::min<int64_t>(1024, (n_out + 256) / 256))),
                       dim3(256), 0, st, hist, n_out + 1, 0);
    const int nb = global_hist_blocks(E);
    hipLaunchKernelGGL((hist_kernel<false>), dim3(nb), dim3(kEvThreads), 0, st, index, E, n_out, 1, hist, errs,
                       ticket, flags, n_scan + 1);
    n_err = nb;
  }
  hipLaunchKernelGGL(scan_kernel, dim3(static_cast<unsigned>(n_scan)), dim3(kScanCells * kScanTpc), 0, st, hist,
                     L.n_hist, n_out, off, ticket, flags, errs, n_err, status);
  if (lds) {
    hipLaunchKernelGGL((bucket_kernel<true>), dim3(L.n_hist), dim3(kEvThreads), 0, st, index, E, n_out, L.n_hist,
                       off, hist, perm);
  } else {
    const int nb = global_hist_blocks(E);
    hipLaunchKernelGGL((bucket_kernel<false>), dim3(nb), dim3(kEvThreads), 0, st, index, E, n_out, 1, off, hist,
                       perm);
  }
  segments(seg_reduce_kernel<MEAN, true>, seg_fixup_kernel<MEAN, true>, perm, off + n_out);
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
  const hipError_t e = ssla::read_to_host(&v, workspace, sizeof(int32_t), st);
  if (e != hipSuccess) {
    ssla::set_error("scatter_check: %s", hipGetErrorString(e));
    return SSLA_ERR_LAUNCH;
  }
  *status_out = v;
  return SSLA_OK;
}
