// Scatter-reduce along dim 0 with an index broadcast over channels:
// torch_scatter.scatter_max / scatter_mean as called by SparsePool.forward
// (reference layers/sparse_pooling.py:33; torch_scatter itself is an
// un-vendored dependency, so the semantics implemented are its documented
// ones: empty rows give 0 (max: argmax = E), mean = sum / max(count, 1)).
//
// Two pipelines, all on the caller's stream, no host synchronisation, no
// memset:
//
// Sorted index (the reference's own call: segment ids from
// unique_consecutive are non-decreasing):   seg_range -> seg_link
// * seg_range: one workgroup of 8 wavefronts per range of 512 positions
//   (every workgroup the same size of work, however the rows are spread).
//   Each wavefront walks a contiguous part of 64 positions as one batch
//   (lane = channel: each position is one coalesced row load, 64 in flight
//   at once) and writes the rows that start and end inside its part;
//   rows that cross a wavefront edge are merged through LDS; a row that
//   crosses the workgroup's start or end leaves one 512-byte piece, and every
//   workgroup writes its tail flag (state, row, event count, bad-index bit).
// * seg_link: one wavefront per range; a range whose last row continues
//   reads the flags of the ranges after it (64 at a time), folds the pieces
//   of the row in range order and writes it; also raises the status word for
//   a bad index.  At C4 there are ~2,000 range edges and most rows end
//   inside their range, so the link is a small pass.
//
// Unsorted index:   hist -> scan -> bucket -> bucket_reduce
// * hist  : LDS histogram of buckets of 64 consecutive rows per event range
//           (a few hundred buckets, so the histogram is small and the
//           workgroups many).
// * scan  : per-bucket start offsets (and per-workgroup offsets inside each
//           bucket) and the prefix of each bucket's chunk count, by a
//           single-pass decoupled look-back; both counts travel in the flag
//           word.  It also writes one descriptor per chunk (bucket, first
//           and last position, chunks of the bucket).
// * bucket: (event, row) pairs placed at their bucket-grouped positions.
// * bucket_reduce: one workgroup per chunk of at most 1792 events of one
//           bucket (its descriptor is one load; full chunks run first and
//           each bucket's partial last chunk in the grid's last round): a
//           64-row x 64-channel tile in LDS takes every event with
//           LDS atomics (max: ds_max_u64 on a packed (orderable value,
//           inverted event id) key, so the result does not depend on the
//           order the events arrive in; mean: ds_add_f64 and a row count).
//           A bucket of one chunk is written out directly; the chunks of a
//           larger bucket leave their tiles (device-scope stores) and count
//           themselves in on a per-bucket counter that hist cleared, and
//           the last to arrive folds the others' tiles into its own and
//           writes the rows (no spin: nothing ever waits on another chunk).
// Max/argmax select (value, smallest event id), NaN never wins, -0.0 ties
// +0.0 and out keeps the sign of the winner's zero: bit-exact and
// deterministic on both paths.  Mean sums in fp64 and rounds once (the
// unsorted path's fp64 sum order follows the LDS atomics, so its last fp64
// bits may vary between runs).
#include "common.h"

namespace ssla {
namespace {

#ifndef SSLA_SR_CHUNK
#define SSLA_SR_CHUNK 1792
#endif
#ifndef SSLA_SR_RANGE
#define SSLA_SR_RANGE 512
#endif
constexpr int kBucketShift = 6;                    // 64 output rows per bucket
constexpr int kBucketRows = 1 << kBucketShift;
constexpr int kEvThreads = 1024;                   // hist / bucket workgroup size
constexpr int kMaxHist = 256;                      // histogram rows (workgroups) at most
constexpr int kEvPerBlock = 4096;                  // events per histogram workgroup (target)
constexpr int kLdsBuckets = 4096;                  // buckets counted in LDS (16 KB); more: global counters
constexpr int kScanCells = 64;                     // buckets per scan workgroup
constexpr int kScanTpc = 1024 / kScanCells;        // scan threads per bucket
constexpr int kChunk = SSLA_SR_CHUNK;              // events per bucket_reduce workgroup at most
#ifndef SSLA_SR_REDW
#define SSLA_SR_REDW 16
#endif
constexpr int kRedWaves = SSLA_SR_REDW;            // bucket_reduce wavefronts
#ifndef SSLA_SR_RWAVES
#define SSLA_SR_RWAVES 8
#endif
constexpr int kRangeWaves = SSLA_SR_RWAVES;        // seg_range wavefronts
constexpr int kRange = SSLA_SR_RANGE;              // positions per seg_range workgroup
constexpr int kPart = kRange / kRangeWaves;        // positions per seg_range wavefront
static_assert(kPart % 64 == 0, "a wavefront part is whole batches of 64 positions");
constexpr int kLinkWaves = 4;

inline int64_t n_buckets(int64_t n_out) { return (n_out + kBucketRows - 1) >> kBucketShift; }
inline int64_t n_ranges(int64_t E) { return std::max<int64_t>(1, (E + kRange - 1) / kRange); }
inline int64_t n_chunks_max(int64_t E, int64_t NB) { return NB + (E + kChunk - 1) / kChunk; }

struct WsLayout {
  size_t status, errs, off, coff, cdesc, flags, hist, perm, parts, pcnt, arrive, rflags, rpieces, total;
  int n_hist;
  int64_t NB, n_chunks, n_rseg;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

inline bool lds_hist(int64_t NB) { return NB <= kLdsBuckets; }

inline int hist_rows(int64_t E, int64_t NB) {
  if (!lds_hist(NB)) return 1;   // global-atomic counting (buckets too many for LDS)
  const int64_t r = (E + kEvPerBlock - 1) / kEvPerBlock;
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kMaxHist, r)));
}

inline int64_t scan_blocks(int64_t NB) { return (NB + kScanCells - 1) / kScanCells; }

// Histogram workgroups of the global-counter mode (also their error slots).
inline int global_hist_blocks(int64_t E) {
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(1024, (E + kEvThreads - 1) / kEvThreads)));
}

inline WsLayout ws_layout(int64_t E, int C, int64_t n_out) {
  WsLayout L;
  L.NB = std::max<int64_t>(1, n_buckets(n_out));
  L.n_hist = hist_rows(E, L.NB);
  L.n_chunks = n_chunks_max(E, L.NB);
  const int64_t ncb = (C + 63) / 64;
  L.n_rseg = n_ranges(E) * ncb;
  const int n_err = std::max(L.n_hist, global_hist_blocks(E));
  size_t p = 0;
  L.status = p; p += 256;   // [0] status word, [1] scan ticket
  L.errs = p;  p = align256(p + sizeof(int32_t) * n_err);
  L.off = p;   p = align256(p + sizeof(int32_t) * (L.NB + 1));
  L.coff = p;  p = align256(p + sizeof(int32_t) * (L.NB + 1));
  L.cdesc = p; p = align256(p + sizeof(int4) * static_cast<size_t>(L.n_chunks));   // (bucket, p0, p1, chunks)
  L.flags = p; p = align256(p + sizeof(uint64_t) * (scan_blocks(L.NB) + 1));
  L.hist = p;  p = align256(p + sizeof(int32_t) * static_cast<size_t>(L.n_hist) * (L.NB + 1));
  L.perm = p;  p = align256(p + sizeof(int2) * (E > 0 ? E : 1));   // (event, row) per bucket-grouped position
  // per (chunk, channel block): a 64 x 64 tile of 8-byte keys / fp64 sums;
  // per chunk: 64 row counts
  L.parts = p; p = align256(p + sizeof(uint64_t) * static_cast<size_t>(L.n_chunks) * ncb * 64 * 64);
  L.pcnt = p;  p = align256(p + sizeof(int32_t) * static_cast<size_t>(L.n_chunks) * 64);
  // per (bucket, channel block): chunks of the bucket that have left their tile
  L.arrive = p; p = align256(p + sizeof(int32_t) * static_cast<size_t>(L.NB) * ncb);
  // per (range, channel block): tail flag and head count, tail and head pieces
  L.rflags = p; p = align256(p + sizeof(uint64_t) * 2 * static_cast<size_t>(L.n_rseg));
  L.rpieces = p; p = align256(p + sizeof(uint64_t) * 2 * 64 * static_cast<size_t>(L.n_rseg));
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

// Clears the scan ticket, the look-back flags and the chunk arrival
// counters (kernel 1 of the unsorted pipeline).
__device__ __forceinline__ void clear_scan_state(int32_t *ticket, uint64_t *flags, int64_t n_flags,
                                                 int32_t *arrive, int64_t n_arrive) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *ticket = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_flags; i += stride)
    flags[i] = 0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_arrive; i += stride)
    arrive[i] = 0;
}

// 64-bit value of lane k (a scalar)
__device__ __forceinline__ uint64_t rl64(uint64_t v, int k) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int32_t>(v), k));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int32_t>(v >> 32), k));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// ---------------------------------------------------------------- hist --
// LDS mode: row b of hist = bucket counts of the events of range b.
// Global mode (more buckets than LDS holds): one shared row of global
// counters, which the preceding fill kernel cleared.
template <bool LDS>
__global__ __launch_bounds__(kEvThreads) void hist_kernel(
    const int64_t *__restrict__ index, int64_t E, int64_t n_out, int64_t NB, int n_hist,
    int32_t *__restrict__ hist, int32_t *__restrict__ errs, int32_t *ticket, uint64_t *flags,
    int64_t n_flags, int32_t *arrive, int64_t n_arrive) {
  clear_scan_state(ticket, flags, n_flags, arrive, n_arrive);
  bool bad = false;
  if constexpr (LDS) {
    __shared__ int32_t lh[kLdsBuckets];
    for (int64_t c = threadIdx.x; c < NB; c += kEvThreads) lh[c] = 0;
    __syncthreads();
    int64_t e0, e1;
    event_range(E, n_hist, blockIdx.x, e0, e1);
    // up to eight index loads per thread in flight at once (a range of
    // 4096 events is four per thread: one round trip, not four)
    for (int64_t e = e0 + threadIdx.x; e < e1; e += 8 * kEvThreads) {
      int64_t r[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) r[u] = e + u * kEvThreads < e1 ? index[e + u * kEvThreads] : 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (e + u * kEvThreads >= e1) break;
        if (bad_row(r[u], n_out)) bad = true;
        else atomicAdd(&lh[r[u] >> kBucketShift], 1);
      }
    }
    __syncthreads();
    int32_t *row = hist + static_cast<int64_t>(blockIdx.x) * (NB + 1);
    for (int64_t c = threadIdx.x; c < NB; c += kEvThreads) row[c] = lh[c];
  } else {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kEvThreads;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kEvThreads + threadIdx.x; e < E; e += stride) {
      const int64_t r = index[e];
      if (bad_row(r, n_out)) bad = true;
      else atomicAdd(&hist[r >> kBucketShift], 1);
    }
  }
  const int any_bad = __syncthreads_or(bad ? 1 : 0);
  if (threadIdx.x == 0) errs[blockIdx.x] = any_bad ? SSLA_ERR_ARG : SSLA_OK;
}

// ---------------------------------------------------------------- scan --
// Look-back word: [63:62] state (0 none, 1 aggregate, 2 inclusive prefix),
// [61:31] chunk count, [30:0] event count.  Counts saturate at 2^31 - 1, so
// inconsistent input can give wrong offsets but never touches the state
// bits, and the look-back always terminates.
constexpr uint64_t kFlagAgg = 1ull << 62, kFlagIncl = 2ull << 62;
constexpr uint64_t kMask31 = 0x7fffffffull;

__device__ __forceinline__ uint64_t pack_counts(int64_t cnt, int64_t chk) {
  const uint64_t a = static_cast<uint64_t>(min(max(cnt, (int64_t)0), (int64_t)kMask31));
  const uint64_t b = static_cast<uint64_t>(min(max(chk, (int64_t)0), (int64_t)kMask31));
  return (b << 31) | a;
}

// Descriptor slot of chunk j of bucket b (ok: chunks of the buckets before
// it, nch: its chunks, n_slots: the grid's slots): the full chunks of all
// buckets at the bottom in bucket order (ok - b counts the full chunks
// before bucket b), each bucket's last, partial chunk at n_slots - 1 - b.
// The reduce grid therefore runs the full chunks first and the
// partial ones in its last round.
__host__ __device__ __forceinline__ int64_t chunk_slot(int64_t b, int64_t ok, int64_t j, int64_t nch,
                                                       int64_t n_slots) {
  return j + 1 < nch ? ok - b + j : n_slots - 1 - b;
}

// Chunks of a bucket of n events: at least one (so every bucket, empty or
// not, has a workgroup that writes its rows).
__device__ __forceinline__ int64_t bucket_chunks(int64_t n) { return max((n + kChunk - 1) / kChunk, (int64_t)1); }

// Counts are column sums of the [n_hist, NB] histogram matrix; each column
// is rewritten with its exclusive prefix (the start offset of each histogram
// workgroup inside the bucket); off = exclusive prefix of the counts over
// buckets (off[NB] = events kept) and coff = that of the chunk counts
// (coff[NB] = chunks).
__global__ __launch_bounds__(kScanCells *kScanTpc) void scan_kernel(
    int32_t *__restrict__ hist, int n_hist, int64_t NB, int32_t *__restrict__ off, int32_t *__restrict__ coff,
    int4 *__restrict__ cdesc, int64_t n_cmax, int32_t *ticket, uint64_t *flags, const int32_t *__restrict__ errs,
    int n_err, int32_t *__restrict__ status) {
  __shared__ int s_bid;
  __shared__ int32_t s_part[kScanTpc][kScanCells];
  __shared__ int64_t s_cnt[kScanCells], s_chk[kScanCells];
  __shared__ int64_t s_wc[kScanCells / 64], s_wk[kScanCells / 64];
  __shared__ int64_t s_excl, s_excl_chk;
  const int tid = threadIdx.x;
  if (tid == 0) s_bid = atomicAdd(ticket, 1);
  __syncthreads();
  const int64_t bid = s_bid;
  const int lc = tid % kScanCells, grp = tid / kScanCells;
  const int64_t cell = bid * kScanCells + lc;
  const bool live = cell < NB;

  // column segment [b0, b1) of this thread
  constexpr int kPer = (kMaxHist + kScanTpc - 1) / kScanTpc;
  const int per = (n_hist + kScanTpc - 1) / kScanTpc;
  const int b0 = min(n_hist, grp * per), b1 = min(n_hist, b0 + per);
  int32_t v[kPer];
  int32_t sum = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    v[i] = (live && b0 + i < b1) ? hist[static_cast<int64_t>(b0 + i) * (NB + 1) + cell] : 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) sum += v[i];
  s_part[grp][lc] = sum;
  __syncthreads();
  int32_t run = 0;
  for (int g2 = 0; g2 < grp; ++g2) run += s_part[g2][lc];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (live && b0 + i < b1) hist[static_cast<int64_t>(b0 + i) * (NB + 1) + cell] = run;
    run += v[i];
  }
  if (grp == kScanTpc - 1) {   // column total
    s_cnt[lc] = run;
    s_chk[lc] = live ? bucket_chunks(run) : 0;
  }
  __syncthreads();
  // inclusive scans over the block's buckets: wavefront scans, then carries
  int64_t c = 0, k = 0;
  if (tid < kScanCells) {
    c = s_cnt[tid];
    k = s_chk[tid];
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t c2 = __shfl_up(c, d);
      const int64_t k2 = __shfl_up(k, d);
      if ((tid & 63) >= d) {
        c += c2;
        k += k2;
      }
    }
    if ((tid & 63) == 63) {
      s_wc[tid >> 6] = c;
      s_wk[tid >> 6] = k;
    }
  }
  __syncthreads();
  if (tid < kScanCells) {
    for (int q = 0; q < (tid >> 6); ++q) {
      c += s_wc[q];
      k += s_wk[q];
    }
    s_cnt[tid] = c;
    s_chk[tid] = k;
  }
  __syncthreads();
  // Windowed look-back by the first wavefront: lane l reads the flag of
  // block bid-1-l; the walk stops at the nearest inclusive prefix.  The
  // payload travels inside the flag word, so relaxed agent-scope atomics
  // suffice (no fences, which would write back / invalidate the L2).
  if (tid < 64) {
    const int64_t agg = s_cnt[kScanCells - 1], agg_k = s_chk[kScanCells - 1];
    int64_t ex = 0, ex_k = 0;
    if (bid > 0) {
      if (tid == 0)
        __hip_atomic_store(&flags[bid], kFlagAgg | pack_counts(agg, agg_k), __ATOMIC_RELAXED,
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
        int64_t vc = tid <= last ? static_cast<int64_t>(w & kMask31) : 0;
        int64_t vk = tid <= last ? static_cast<int64_t>((w >> 31) & kMask31) : 0;
        for (int d = 32; d >= 1; d >>= 1) {
          vc += __shfl_xor(vc, d);
          vk += __shfl_xor(vk, d);
        }
        ex += vc;
        ex_k += vk;
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
      __hip_atomic_store(&flags[bid], kFlagIncl | pack_counts(ex + agg, ex_k + agg_k), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      s_excl = ex;
      s_excl_chk = ex_k;
      if (bid == static_cast<int64_t>(gridDim.x) - 1) {
        off[NB] = static_cast<int32_t>(ex + agg);
        coff[NB] = static_cast<int32_t>(ex_k + agg_k);
      }
    }
  }
  __syncthreads();
  if (live) {
    const int64_t mine = lc > 0 ? s_cnt[lc] - s_cnt[lc - 1] : s_cnt[0];
    const int64_t mine_k = lc > 0 ? s_chk[lc] - s_chk[lc - 1] : s_chk[0];
    const int64_t o = s_excl + s_cnt[lc] - mine, ok = s_excl_chk + s_chk[lc] - mine_k;
    if (grp == 0) {
      off[cell] = static_cast<int32_t>(o);
      coff[cell] = static_cast<int32_t>(ok);
    }
    // the bucket's chunk descriptors: a reduce workgroup finds its bucket
    // and positions in one load.  Full chunks fill the slots from the
    // bottom, every bucket's last (partial) chunk the slots from the top
    // (chunk_slot), so the reduce grid runs the full chunks first.
    for (int64_t j = grp; j < mine_k; j += kScanTpc) {
      const int64_t p0 = o + j * kChunk, p1 = min(p0 + static_cast<int64_t>(kChunk), o + mine);
      const int64_t slot = chunk_slot(cell, ok, j, mine_k, n_cmax);
      if (slot >= 0 && slot < n_cmax)
        cdesc[slot] = make_int4(static_cast<int>(cell), static_cast<int>(p0), static_cast<int>(p1),
                                static_cast<int>(mine_k));
    }
  }
}

// -------------------------------------------------------------- bucket --
// perm[off[b] + start of this workgroup in bucket b + rank] = (e, row): one
// 8-byte store per event.
template <bool LDS>
__global__ __launch_bounds__(kEvThreads) void bucket_kernel(
    const int64_t *__restrict__ index, int64_t E, int64_t n_out, int64_t NB, int n_hist,
    const int32_t *__restrict__ off, int32_t *__restrict__ hist, int2 *__restrict__ perm) {
  if constexpr (LDS) {
    __shared__ int32_t lc[kLdsBuckets];
    const int32_t *row = hist + static_cast<int64_t>(blockIdx.x) * (NB + 1);
    for (int64_t c = threadIdx.x; c < NB; c += kEvThreads) lc[c] = off[c] + row[c];
    __syncthreads();
    int64_t e0, e1;
    event_range(E, n_hist, blockIdx.x, e0, e1);
    // up to eight index loads per thread in flight at once, as in hist
    for (int64_t e = e0 + threadIdx.x; e < e1; e += 8 * kEvThreads) {
      int64_t r[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) r[u] = e + u * kEvThreads < e1 ? index[e + u * kEvThreads] : -1;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (e + u * kEvThreads >= e1) break;
        if (bad_row(r[u], n_out)) continue;
        const int32_t pos = atomicAdd(&lc[r[u] >> kBucketShift], 1);
        if (pos >= 0 && pos < E) perm[pos] = make_int2(static_cast<int32_t>(e + u * kEvThreads), static_cast<int32_t>(r[u]));
      }
    }
  } else {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kEvThreads;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kEvThreads + threadIdx.x; e < E; e += stride) {
      const int64_t r = index[e];
      if (bad_row(r, n_out)) continue;
      const int64_t b = r >> kBucketShift;
      const int32_t pos = off[b] + atomicAdd(&hist[b], 1);
      if (pos >= 0 && pos < E) perm[pos] = make_int2(static_cast<int32_t>(e), static_cast<int32_t>(r));
    }
  }
}

// ---------------------------------------------------------- max / mean --
// Order-independent max key of (value x, event e): the value's bits made
// unsigned-orderable (-0.0 taken as +0.0) in the high word; in the low word
// the inverted event id (so the smallest id wins a tie) above the sign of a
// zero (so the winner's -0.0 comes back).  E < 2^31.  The event part
// lo_base = (0x7fffffff - e) << 1 is wavefront-uniform (the scalar unit
// forms it).  NaN values have no key: the caller leaves them out of the
// maximum (key 0 would mean the same: every event beats it), so NaN never
// wins and a row with no winner reads 0.
__device__ __forceinline__ uint64_t max_key_part(float x, uint32_t lo_base) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t u0 = x != 0.f ? u : 0u;   // -0 folded onto +0
  const uint32_t m = static_cast<uint32_t>(static_cast<int32_t>(u0) >> 31);
  const uint32_t ord = u0 ^ (m | 0x80000000u);   // negative: ~u0, else u0 | sign bit
  const uint32_t lo = lo_base | ((u ^ u0) >> 31);   // the low bit: x was -0
  return (static_cast<uint64_t>(ord) << 32) | lo;
}
// (value, event) of a key != 0
__device__ __forceinline__ void key_value(uint64_t key, float &x, int64_t &e) {
  const uint32_t ord = static_cast<uint32_t>(key >> 32);
  const uint32_t lo = static_cast<uint32_t>(key);
  uint32_t u = (ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord;
  if (lo & 1u) u = 0x80000000u;
  x = __uint_as_float(u);
  e = static_cast<int64_t>(0x7fffffffu - (lo >> 1));
}

// Walk accumulators of the sorted path: (value, smallest event id) maximum
// by comparison (NaN never wins: -1 as unsigned is above every event id),
// or an fp64 sum.
template <bool MEAN>
struct SegAcc;
template <> struct SegAcc<false> {
  float best;
  int32_t idx;   // -1: no event yet
  __device__ __forceinline__ void reset() { best = -INFINITY; idx = -1; }
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

// Rows [r0, r1) (clamped to the output) of one channel written as empty.
template <bool MEAN>
__device__ __forceinline__ void seg_empty_rows(float *out, int64_t *argmax, int64_t r0, int64_t r1, int64_t n_out,
                                               int C, int col, bool act, int64_t E) {
  r0 = max(r0, (int64_t)0);
  r1 = min(r1, n_out);
  if (!act) return;
  for (int64_t r = r0; r < r1; ++r) {
    out[r * C + col] = 0.f;
    if constexpr (!MEAN) argmax[r * C + col] = E;
  }
}

// ------------------------------------------------------------ seg_range --
// Range flag (tail flag): bits 62-63 state (0: the range's last row ends at
// the range's end or inside it; 1: the whole range is one row that began
// before it and continues after it; 2: the last row continues past the end:
// a tail piece), bit 61 a bad index seen in the range, bits 31-60 the row
// (clamped, n_out < 2^30), bits 0-30 the events of the tail piece (or of the
// range when state 1).  The second flag word of a range is its head count
// (events of its first row's piece, when that row began before it).
constexpr uint64_t kSegThrough = 1ull << 62, kSegPiece = 2ull << 62, kSegBad = 1ull << 61;
__device__ __forceinline__ uint64_t seg_state(uint64_t f) { return f >> 62; }
__device__ __forceinline__ int64_t seg_row(uint64_t f) { return static_cast<int64_t>((f >> 31) & 0x3fffffffu); }
__device__ __forceinline__ int64_t seg_count(uint64_t f) { return static_cast<int64_t>(f & 0x7fffffffu); }

// wavefront part flags (LDS)
constexpr int kPartLive = 1, kPartOpenStart = 2, kPartOpenEnd = 4, kPartThrough = 8;

constexpr int kRsrcWord3 = 0x00020000;   // raw 32-bit data, range checked
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Buffer resource over [base, base + bytes): loads past the end read 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                           static_cast<int>(min(max(bytes, (int64_t)0), (int64_t)0x7fffffff)),
                                           kRsrcWord3);
}

// A row index saturated to int32: -1 below the output, n_out above it (both
// bad); distinct valid rows stay distinct, so every boundary and order test
// agrees between the workgroups that look at the same positions.
__device__ __forceinline__ int32_t sat_row(int64_t r, int32_t n_out) {
  return r < 0 ? -1 : (r >= n_out ? n_out : static_cast<int32_t>(r));
}

// CT: the channel count at compile time (64: one channel block, row
// offsets become immediates) or 0 (any C, channel blocks of 64).
template <bool MEAN, int CT>
__global__ __launch_bounds__(64 * kRangeWaves) void seg_range_kernel(
    const float *__restrict__ src, const int64_t *__restrict__ index, int32_t E, int C, int32_t n_out,
    float *__restrict__ out, int64_t *__restrict__ argmax, uint64_t *__restrict__ rflags,
    uint64_t *__restrict__ rpieces, int32_t n_rseg, int32_t *__restrict__ status) {
  __shared__ uint64_t s_head[kRangeWaves][64], s_tail[kRangeWaves][64];
  __shared__ int32_t s_hcnt[kRangeWaves], s_tcnt[kRangeWaves], s_trow[kRangeWaves], s_fl[kRangeWaves];
  const int Cc = CT ? CT : C;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int ncb = CT ? 1 : (C + 63) / 64;
  const int rg = static_cast<int>(blockIdx.x) / ncb;
  const int cb = static_cast<int>(blockIdx.x) - rg * ncb;
  const int seg = static_cast<int>(blockIdx.x);   // this workgroup's flags / pieces
  const int col = cb * 64 + lane;
  const bool act = CT ? true : col < C;
  if (blockIdx.x == 0 && threadIdx.x == 0) *status = SSLA_OK;   // bad indices are raised by seg_link
  if (E == 0) {   // no events: every row is empty
    if (w == 0) seg_empty_rows<MEAN>(out, argmax, 0, n_out, n_out, Cc, col, act, E);
    return;
  }
  const int s0 = rg * kRange, s1 = min(s0 + kRange, E);
  const int pa = min(s0 + w * kPart, s1), pb = min(pa + kPart, s1);
  // the range's rows of this channel block and its indices: loads past the
  // range read 0 (and are never used)
  const __amdgpu_buffer_rsrc_t rs_src =
      make_rsrc(src + static_cast<int64_t>(s0) * Cc + cb * 64, (static_cast<int64_t>(s1 - s0) * Cc - cb * 64) * 4);
  const __amdgpu_buffer_rsrc_t rs_idx = make_rsrc(index + s0, static_cast<int64_t>(s1 - s0) * 8);

  auto store_row = [&](int32_t r, const SegAcc<MEAN> &a, int32_t cnt) __attribute__((always_inline)) {
    if (act) seg_store<MEAN>(out, argmax, static_cast<int64_t>(min(max(r, 0), n_out - 1)) * Cc + col, a, cnt, E);
  };

  int fl = 0;
  bool bad = false;
  SegAcc<MEAN> acc, head;
  acc.reset();
  head.reset();
  int32_t cnt = 0, hcnt = 0, cur = 0;
  if (pa < pb) {
    fl = kPartLive;
    const int32_t prev = pa > 0 ? sat_row(index[pa - 1], n_out) : -1;
    const bool open_start = pa > 0 && sat_row(index[pa], n_out) == prev;
    bool in_head = open_start;   // the walk is still in a row that began before this part
    if (open_start) fl |= kPartOpenStart;
    // the open row (open start), or the row before the part: a part that
    // starts a row writes the empty rows between that row and its first
    cur = prev;
    int32_t rlast = prev;   // row of the position before the batch
    auto close_row = [&]() __attribute__((always_inline)) {
      if (cnt > 0) {
        if (in_head) {
          head = acc;
          hcnt = cnt;
          in_head = false;
        } else {
          store_row(cur, acc, cnt);
        }
      }
    };
    for (int s = pa; s < pb; s += 64) {
      const int ne = min(64, pb - s);
      // the 64 row loads first (they do not depend on the index), then the
      // index: one memory round trip per batch, not two
      const uint32_t vb = static_cast<uint32_t>(s - s0) * static_cast<uint32_t>(Cc * 4) + lane * 4u;
      float xr[64];
#pragma unroll
      for (int e = 0; e < 64; ++e)
        xr[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs_src, vb + e * (Cc * 4), 0, 0));
      asm volatile("" ::: "memory");   // the row loads stay ahead of the index load
      const u32x2 raw = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_idx, static_cast<uint32_t>(s - s0 + lane) * 8u, 0, 0));
      const int32_t rr = sat_row(static_cast<int64_t>((static_cast<uint64_t>(raw.y) << 32) | raw.x), n_out);
      const int32_t rup = __shfl_up(rr, 1);   // every lane active
      const int32_t rbefore = lane == 0 ? rlast : rup;
      if (lane < ne && (rr < 0 || rr >= n_out || rr < rbefore)) bad = true;
      // positions where a new row starts; the part's first position starts
      // one unless the part is open at its start
      bool st = lane < ne && rr != rbefore;
      if (s == pa && lane == 0) st = !open_start;
      const uint64_t bnd = __builtin_amdgcn_ballot_w64(st);
      const int32_t rfirst_before = s == pa ? prev : rlast;   // row before the batch
      rlast = __builtin_amdgcn_readlane(rr, ne - 1);
      // eight positions per step; a step without a row start (the common
      // case) runs without any per-position test
#pragma unroll
      for (int e8 = 0; e8 < 64; e8 += 8) {
        if (e8 >= ne) break;
        const uint32_t bb = static_cast<uint32_t>(bnd >> e8) & 0xffu;
        if (bb == 0 && e8 + 8 <= ne) {
#pragma unroll
          for (int k = 0; k < 8; ++k) acc.add(xr[e8 + k], s + e8 + k);
          cnt += 8;
          continue;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int e = e8 + k;
          if (e < ne) {
            if ((bb >> k) & 1) {   // wavefront-uniform: a new row starts at position s + e
              close_row();
              cur = __builtin_amdgcn_readlane(rr, e);
              acc.reset();
              cnt = 0;
            }
            acc.add(xr[e], s + e);
            ++cnt;
          }
        }
      }
      // empty rows between consecutive rows of the batch (and between the
      // row before it and its first), after the walk: one loop, not one per
      // unrolled position
      for (uint64_t m = bnd; m != 0; m &= m - 1) {
        const int e = static_cast<int>(__builtin_ctzll(m));
        const int32_t q = e == 0 ? rfirst_before : __builtin_amdgcn_readlane(rr, e - 1);
        const int32_t r = __builtin_amdgcn_readlane(rr, e);
        if (r > q + 1) seg_empty_rows<MEAN>(out, argmax, static_cast<int64_t>(q) + 1, r, n_out, Cc, col, act, E);
      }
    }
    const bool open_end = pb < E && sat_row(index[pb], n_out) == rlast;
    if (open_end) {
      fl |= kPartOpenEnd | (in_head ? kPartThrough : 0);
    } else {
      close_row();
      if (pb == E) seg_empty_rows<MEAN>(out, argmax, static_cast<int64_t>(cur) + 1, n_out, n_out, Cc, col, act, E);
    }
  }
  s_head[w][lane] = head.pack();
  s_tail[w][lane] = acc.pack();
  if (lane == 0) {
    s_fl[w] = fl;
    s_hcnt[w] = hcnt;
    s_tcnt[w] = cnt;
    s_trow[w] = cur;
  }
  const int any_bad = __syncthreads_or(bad ? 1 : 0);
  if (w != 0) return;
  // ---- fold the parts in order (wavefront 0) ----------------------------
  // `run` is the row open between parts; `from_start` says it began before
  // this range (then it is the range's head piece, or with no end inside the
  // range, the whole range).
  SegAcc<MEAN> run;
  run.reset();
  int32_t rcnt = 0, rrow = 0;
  bool from_start = (s_fl[0] & kPartOpenStart) != 0;
  int last_fl = 0;
  uint64_t *tails = rpieces, *heads = rpieces + static_cast<int64_t>(n_rseg) * 64;
  for (int ww = 0; ww < kRangeWaves; ++ww) {
    const int f = s_fl[ww];
    if (!(f & kPartLive)) break;   // parts past the range's end
    last_fl = f;
    if (f & kPartThrough) {        // the whole part continues the open row
      run.merge(s_tail[ww][lane]);
      rcnt += s_tcnt[ww];
      continue;
    }
    if (f & kPartOpenStart) {      // the open row ends inside this part
      run.merge(s_head[ww][lane]);
      rcnt += s_hcnt[ww];
      if (from_start) {
        heads[static_cast<int64_t>(seg) * 64 + lane] = run.pack();
        if (lane == 0) rflags[n_rseg + seg] = static_cast<uint64_t>(rcnt);
      } else {
        store_row(rrow, run, rcnt);
      }
      from_start = false;
    }
    if (f & kPartOpenEnd) {
      run.reset();
      run.merge(s_tail[ww][lane]);
      rcnt = s_tcnt[ww];
      rrow = s_trow[ww];
    }
  }
  uint64_t tf = any_bad ? kSegBad : 0;
  if (last_fl & kPartOpenEnd) {
    tails[static_cast<int64_t>(seg) * 64 + lane] = run.pack();
    tf |= (from_start ? kSegThrough : kSegPiece) | (static_cast<uint64_t>(min(max(rrow, 0), n_out - 1)) << 31) |
          static_cast<uint64_t>(rcnt);
  }
  if (lane == 0) rflags[seg] = tf;
}

// One wavefront per (range, channel block): a range whose last row
// continues (state 2) folds the row's pieces -- its tail piece, the ranges
// the row runs through (state 1) and the head piece of the range where it
// ends -- in range order and writes the row.  Raises the status word for a
// bad index.
template <bool MEAN>
__global__ __launch_bounds__(64 * kLinkWaves) void seg_link_kernel(int64_t E, int C, int64_t n_out,
                                                                   float *__restrict__ out,
                                                                   int64_t *__restrict__ argmax,
                                                                   const uint64_t *__restrict__ rflags,
                                                                   const uint64_t *__restrict__ rpieces,
                                                                   int64_t n_rng, int32_t *__restrict__ status) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int ncb = (C + 63) / 64;
  const int64_t n_rseg = n_rng * ncb;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * kLinkWaves + w;
  if (E == 0 || q >= n_rseg) return;   // wavefront-uniform
  const int64_t rg = q / ncb;
  const int cb = static_cast<int>(q - rg * ncb);
  const uint64_t f = rflags[q];
  if ((f & kSegBad) && lane == 0) *status = SSLA_ERR_ARG;
  if (seg_state(f) != 2) return;
  const uint64_t *tails = rpieces, *heads = rpieces + n_rseg * 64;
  // te: the first range after rg that is not wholly the row
  int64_t te = n_rng - 1;
  for (int64_t j0 = rg + 1; j0 < n_rng; j0 += 64) {
    const int64_t j = j0 + lane;
    const uint64_t fj = j < n_rng ? rflags[j * ncb + cb] : 0;
    const uint64_t stop = __builtin_amdgcn_ballot_w64(j < n_rng && seg_state(fj) != 1);
    if (stop) {
      te = j0 + static_cast<int64_t>(__builtin_ctzll(stop));
      break;
    }
  }
  SegAcc<MEAN> a;
  a.reset();
  a.merge(tails[q * 64 + lane]);
  int64_t cnt = seg_count(f);
  // the ranges the row runs through, eight pieces in flight per round trip
  // (folded in range order)
  for (int64_t m0 = rg + 1; m0 < te; m0 += 8) {
    uint64_t pc[8], fc[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t m = min(m0 + u, te - 1);
      pc[u] = tails[(m * ncb + cb) * 64 + lane];
      fc[u] = rflags[m * ncb + cb];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (m0 + u < te) {
        a.merge(pc[u]);
        cnt += seg_count(fc[u]);
      }
    }
  }
  if (te > rg) {
    a.merge(heads[(te * ncb + cb) * 64 + lane]);
    cnt += static_cast<int64_t>(rflags[n_rseg + te * ncb + cb] & kMask31);
  }
  const int col = cb * 64 + lane;
  if (col < C) seg_store<MEAN>(out, argmax, seg_row(f) * C + col, a, cnt, E);
}

// ------------------------------------------------------- bucket_reduce --
// One workgroup per (chunk, channel block): the chunk's events (at most
// kChunk consecutive positions of one bucket) go into a 64-row x 64-channel
// LDS tile with LDS atomics.  Wavefronts take batches of kRedBatch positions
// in turn: the batch's (event, row) pairs, then its rows (lane = channel,
// one coalesced 256-byte row load each, all in flight), then one atomic per
// position.  Batches of 32 keep the kernel at two workgroups per CU, so
// every chunk of a config-4 call is resident at once.
#ifndef SSLA_SR_RBATCH
#define SSLA_SR_RBATCH 32
#endif
constexpr int kRedBatch = SSLA_SR_RBATCH;
static_assert(kRedBatch <= 64, "a batch's (event, row) pairs are one per lane");
template <bool MEAN, int CT>
__global__ __launch_bounds__(64 * kRedWaves) void bucket_reduce_kernel(
    const float *__restrict__ src, const int2 *__restrict__ perm, const int4 *__restrict__ cdesc,
    const int32_t *__restrict__ coff, int32_t NB, int32_t E, int C, int32_t n_out, float *__restrict__ out,
    int64_t *__restrict__ argmax, uint64_t *__restrict__ parts, int32_t *__restrict__ pcnt,
    int32_t *__restrict__ arrive, int32_t n_slots) {
  __shared__ uint64_t tile[kBucketRows][64];   // max keys, or fp64 sums
  __shared__ int32_t tcnt[kBucketRows];
  __shared__ int32_t s_last;
  const int Cc = CT ? CT : C;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int ncb = CT ? 1 : (C + 63) / 64;
  const int c = static_cast<int>(blockIdx.x) / ncb;
  const int cb = static_cast<int>(blockIdx.x) - c * ncb;
  // the chunk count and this slot's descriptor in one round trip (the grid
  // covers the most chunks there can be; slots between the full chunks and
  // the buckets' last chunks hold none)
  const int32_t n_chunks = coff[NB];
  const int4 d = cdesc[c];
  if (c >= n_chunks - NB && c < n_slots - NB) return;   // workgroup-uniform
  for (int i = threadIdx.x; i < kBucketRows * 64; i += 64 * kRedWaves) (&tile[0][0])[i] = 0ull;
  if (threadIdx.x < kBucketRows) tcnt[threadIdx.x] = 0;
  __syncthreads();
  const int b = min(max(d.x, 0), NB - 1), nch = d.w;
  const int p0 = min(max(d.y, 0), E);
  const int p1 = min(max(d.z, p0), E);
  const int row0 = b << kBucketShift;
  const int col = cb * 64 + lane;
  const bool act = CT ? true : col < C;
  // this lane's channel (lanes past C re-read the last one, unused)
  const uint32_t colc = static_cast<uint32_t>(CT ? col : min(col, Cc - 1));
  // rows through a buffer resource over src when its bytes fit 31-bit offsets
  const bool rows32 = static_cast<int64_t>(E) * Cc * 4 < 0x7fffffff;
  const __amdgpu_buffer_rsrc_t rs_rows = make_rsrc(src, static_cast<int64_t>(E) * Cc * 4);
  // the (event, row) pairs of this wavefront's next batch are loaded while
  // the current batch's rows are in flight
  int s = p0 + w * kRedBatch;
  int2 pr_next = (s < p1 && lane < min(kRedBatch, p1 - s)) ? perm[s + lane] : make_int2(0, row0);
  for (; s < p1; s += kRedBatch * kRedWaves) {
    const int ne = min(kRedBatch, p1 - s);
    const int2 pr = pr_next;
    const int sn = s + kRedBatch * kRedWaves;
    const int32_t ev = min(max(pr.x, 0), E - 1);
    const int32_t rl = (pr.y - row0) & (kBucketRows - 1);
    float xr[kRedBatch];
    // event ids are wavefront-uniform (read lane by lane): the row offset
    // goes in the scalar offset field, with no address arithmetic per lane
    if (rows32) {
#pragma unroll
      for (int e = 0; e < kRedBatch; ++e)
        xr[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            rs_rows, colc * 4u,
            static_cast<uint32_t>(__builtin_amdgcn_readlane(ev, e)) * static_cast<uint32_t>(Cc * 4), 0));
    } else {
#pragma unroll
      for (int e = 0; e < kRedBatch; ++e)
        xr[e] = src[static_cast<int64_t>(__builtin_amdgcn_readlane(ev, e)) * Cc + colc];
    }
    pr_next = (sn < p1 && lane < min(kRedBatch, p1 - sn)) ? perm[sn + lane] : make_int2(0, row0);
#pragma unroll
    for (int e = 0; e < kRedBatch; ++e) {
      if (e < ne) {
        const int32_t r = __builtin_amdgcn_readlane(rl, e);
        if constexpr (MEAN) {
          if (act) atomicAdd(reinterpret_cast<double *>(&tile[r][lane]), static_cast<double>(xr[e]));
          if (lane == 0) atomicAdd(&tcnt[r], 1);
        } else {
          const uint32_t lo_base = (0x7fffffffu - static_cast<uint32_t>(__builtin_amdgcn_readlane(ev, e))) << 1;
          if (act && !(xr[e] != xr[e]))   // NaN never wins
            atomicMax(reinterpret_cast<unsigned long long *>(&tile[r][lane]),
                      static_cast<unsigned long long>(max_key_part(xr[e], lo_base)));
        }
      }
    }
  }
  __syncthreads();
  if (nch > 1) {
    // One chunk of a larger bucket: leave the tile, written through to
    // device scope (relaxed agent-scope stores), then count this chunk in.
    // The bucket's last chunk to arrive -- on whichever XCD -- folds the
    // others' tiles into its own and writes the rows; the stores are
    // complete before the count, so it reads them all.
    uint64_t *pt = parts + (static_cast<int64_t>(c) * ncb + cb) * (kBucketRows * 64);
    for (int rr = w; rr < kBucketRows; rr += kRedWaves)
      __hip_atomic_store(&pt[rr * 64 + lane], tile[rr][lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (MEAN && cb == 0 && threadIdx.x < kBucketRows)
      __hip_atomic_store(&pcnt[static_cast<int64_t>(c) * kBucketRows + threadIdx.x], tcnt[threadIdx.x],
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this thread's stores are complete
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(&arrive[static_cast<int64_t>(b) * ncb + cb], 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == nch - 1;
    __syncthreads();
    if (!s_last) return;   // workgroup-uniform
  }
  // Write the bucket's rows: this chunk's tile, folded (for a bucket of
  // several chunks) with the other chunks' tiles in chunk order.
  const int ok = nch > 1 ? coff[b] : 0;
  for (int rr = w; rr < kBucketRows; rr += kRedWaves) {
    const int row = row0 + rr;
    if (row >= n_out || !act) continue;
    uint64_t key = MEAN ? 0ull : tile[rr][lane];
    double sum = 0.0;
    int64_t n = 0;
    for (int jj = 0; jj < nch; jj += 4) {   // four tiles' loads in flight
      uint64_t v[4];
      int32_t k[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int ch = nch > 1 ? static_cast<int>(chunk_slot(b, ok, min(jj + u, nch - 1), nch, n_slots)) : c;
        if (ch == c) {
          v[u] = tile[rr][lane];
          k[u] = MEAN ? tcnt[rr] : 0;
        } else {
          v[u] = __hip_atomic_load(&parts[(static_cast<int64_t>(ch) * ncb + cb) * (kBucketRows * 64) + rr * 64 + lane],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          k[u] = MEAN ? __hip_atomic_load(&pcnt[static_cast<int64_t>(ch) * kBucketRows + rr], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT)
                      : 0;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (jj + u < nch) {
          if constexpr (MEAN) {
            sum += __longlong_as_double(static_cast<long long>(v[u]));
            n += k[u];
          } else {
            key = v[u] > key ? v[u] : key;
          }
        }
      }
    }
    const int64_t o = static_cast<int64_t>(row) * Cc + col;
    if constexpr (MEAN) {
      out[o] = n > 0 ? static_cast<float>(sum / static_cast<double>(n)) : 0.f;
    } else {
      float x = 0.f;
      int64_t e = E;
      if (key != 0ull) key_value(key, x, e);
      out[o] = x;
      argmax[o] = e;
    }
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
  const int64_t ncb = (C + 63) / 64;
  // the sorted path addresses each range's rows through a 32-bit buffer
  // resource (kRange rows of C channels)
  SSLA_CHECK_ARG(static_cast<int64_t>(kRange) * C * 4 < 0x7fffffff, "%s: C=%d channels too many", name, C);
  if (sorted) {
    const int64_t n_rng = n_ranges(E);
    uint64_t *rflags = reinterpret_cast<uint64_t *>(base + L.rflags);
    uint64_t *rpieces = reinterpret_cast<uint64_t *>(base + L.rpieces);
    SSLA_CHECK_ARG(L.n_rseg < 0x7fffffff, "%s: too many events x channel blocks", name);
    const int32_t E32 = static_cast<int32_t>(E), n32 = static_cast<int32_t>(n_out), r32 = static_cast<int32_t>(L.n_rseg);
    if (C == 64)
      hipLaunchKernelGGL((seg_range_kernel<MEAN, 64>), dim3(static_cast<unsigned>(L.n_rseg)), dim3(64 * kRangeWaves),
                         0, st, src, index, E32, C, n32, out, argmax, rflags, rpieces, r32, status);
    else
      hipLaunchKernelGGL((seg_range_kernel<MEAN, 0>), dim3(static_cast<unsigned>(L.n_rseg)), dim3(64 * kRangeWaves),
                         0, st, src, index, E32, C, n32, out, argmax, rflags, rpieces, r32, status);
    hipLaunchKernelGGL(seg_link_kernel<MEAN>, dim3(static_cast<unsigned>((L.n_rseg + kLinkWaves - 1) / kLinkWaves)),
                       dim3(64 * kLinkWaves), 0, st, E, C, n_out, out, argmax, rflags, rpieces, n_rng, status);
    return launch_status(name);
  }
  // unsorted: bucketing by 64-row buckets, then the LDS reduce per chunk
  int32_t *errs = reinterpret_cast<int32_t *>(base + L.errs);
  int32_t *off = reinterpret_cast<int32_t *>(base + L.off);
  int32_t *coff = reinterpret_cast<int32_t *>(base + L.coff);
  int4 *cdesc = reinterpret_cast<int4 *>(base + L.cdesc);
  uint64_t *flags = reinterpret_cast<uint64_t *>(base + L.flags);
  int32_t *hist = reinterpret_cast<int32_t *>(base + L.hist);
  int2 *perm = reinterpret_cast<int2 *>(base + L.perm);
  uint64_t *parts = reinterpret_cast<uint64_t *>(base + L.parts);
  int32_t *pcnt = reinterpret_cast<int32_t *>(base + L.pcnt);
  int32_t *arrive = reinterpret_cast<int32_t *>(base + L.arrive);
  const int64_t NB = L.NB;
  const int64_t n_scan = scan_blocks(NB);
  const bool lds = lds_hist(NB);
  SSLA_CHECK_ARG(L.n_chunks * ncb < 0x7fffffff && NB * ncb < 0x7fffffff, "%s: too many chunks x channel blocks",
                 name);
  int n_err = 0;
  if (lds) {
    hipLaunchKernelGGL((hist_kernel<true>), dim3(L.n_hist), dim3(kEvThreads), 0, st, index, E, n_out, NB, L.n_hist,
                       hist, errs, ticket, flags, n_scan + 1, arrive, NB * ncb);
    n_err = L.n_hist;
  } else {
    hipLaunchKernelGGL(fill_i32, dim3(static_cast<unsigned>(std::min<int64_t>(1024, (NB + 256) / 256))), dim3(256),
                       0, st, hist, NB + 1, 0);
    const int nb = global_hist_blocks(E);
    hipLaunchKernelGGL((hist_kernel<false>), dim3(nb), dim3(kEvThreads), 0, st, index, E, n_out, NB, 1, hist, errs,
                       ticket, flags, n_scan + 1, arrive, NB * ncb);
    n_err = nb;
  }
  hipLaunchKernelGGL(scan_kernel, dim3(static_cast<unsigned>(n_scan)), dim3(kScanCells * kScanTpc), 0, st, hist,
                     L.n_hist, NB, off, coff, cdesc, L.n_chunks, ticket, flags, errs, n_err, status);
  if (lds) {
    hipLaunchKernelGGL((bucket_kernel<true>), dim3(L.n_hist), dim3(kEvThreads), 0, st, index, E, n_out, NB,
                       L.n_hist, off, hist, perm);
  } else {
    const int nb = global_hist_blocks(E);
    hipLaunchKernelGGL((bucket_kernel<false>), dim3(nb), dim3(kEvThreads), 0, st, index, E, n_out, NB, 1, off, hist,
                       perm);
  }
  {
    const int32_t E32 = static_cast<int32_t>(E), n32 = static_cast<int32_t>(n_out), NB32 = static_cast<int32_t>(NB);
    if (C == 64)
      hipLaunchKernelGGL((bucket_reduce_kernel<MEAN, 64>), dim3(static_cast<unsigned>(L.n_chunks * ncb)),
                         dim3(64 * kRedWaves), 0, st, src, perm, cdesc, coff, NB32, E32, C, n32, out, argmax, parts,
                         pcnt, arrive, static_cast<int32_t>(L.n_chunks));
    else
      hipLaunchKernelGGL((bucket_reduce_kernel<MEAN, 0>), dim3(static_cast<unsigned>(L.n_chunks * ncb)),
                         dim3(64 * kRedWaves), 0, st, src, perm, cdesc, coff, NB32, E32, C, n32, out, argmax, parts,
                         pcnt, arrive, static_cast<int32_t>(L.n_chunks));
  }
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
