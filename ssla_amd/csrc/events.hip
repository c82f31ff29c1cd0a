// Event-stream glue on gfx950: grouping events by pixel, scattering pixel
// groups into receptive fields / patches, ordered index-add, truncation,
// temporal dropout, pooling keys and the sparse-to-dense grid.
//
// These restate the reference's torch index pipelines
// (utils/farsecnn_utils.py, utils/async_utils.py, layers/sparse_pooling.py,
// layers/temporal_dropout.py, layers/linear_attention.py, model_mos.py) as a
// few fused kernels each.  Device-wide orderings use a stable LSD radix sort
// and prefix sums from rocPRIM (AMD's header library, compiled in here);
// every other step is a kernel of this file.  All sorts are stable: ties keep
// the order in which items were enumerated, which is the order the
// reference produces whenever its own sort is stable.
//
// Calls whose output size depends on the data write their counts into a
// small device array `counts` (int64) of the workspace; the caller reads it
// after the call and uses the leading part of the capacity-sized outputs.
#include <cstring>
#include <rocprim/rocprim.hpp>

#include "common.h"

namespace ssla {
namespace {

constexpr int kThreads = 256;

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
inline unsigned grid_for(int64_t n) {
  return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((n + kThreads - 1) / kThreads, 1 << 20)));
}
#define GRID_STRIDE(i, n)                                                                       \
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < (n);      \
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)

inline int bits_for(uint64_t max_value) {
  int b = 0;
  while (b < 64 && (max_value >> b) != 0) ++b;
  return std::max(b, 1);
}

// Workspace carve-out helper.
struct Carve {
  char *base;
  size_t off = 0;
  template <class T>
  T *take(size_t n) {
    T *p = reinterpret_cast<T *>(base ? base + off : nullptr);
    off = align256(off + sizeof(T) * std::max<size_t>(n, 1));
    return p;
  }
};

// Radix sorts of (8-byte key, 4-byte value) pairs: rocPRIM's merge sort up
// to 2^18 items, its onesweep LSD passes above.  Measured on MI355X
// (µs per sort, 17-bit / 36-bit keys): 20k items 36 / 39 merge against 74 /
// 118 onesweep, 50k 40 / 43 against 76 / 123, 200k 67 / 71 against 81 /
// 131, 500k 138 / 141 against 88 / 140, 1M 183 / 190 against 97 / 155.
using SortConfig = rocprim::radix_sort_config<rocprim::default_config, rocprim::default_config,
                                              rocprim::default_config, (size_t{1} << 18)>;

// rocPRIM temporary storage sizes (queried with a null buffer).
size_t sort_temp_bytes(size_t n) {
  size_t tb = 0;
  rocprim::radix_sort_pairs<SortConfig>(nullptr, tb, static_cast<uint64_t *>(nullptr), static_cast<uint64_t *>(nullptr),
                            static_cast<int32_t *>(nullptr), static_cast<int32_t *>(nullptr), std::max<size_t>(n, 1),
                            0, 64);
  return tb;
}
size_t scan_temp_bytes(size_t n) {
  size_t tb = 0;
  rocprim::exclusive_scan(nullptr, tb, static_cast<int64_t *>(nullptr), static_cast<int64_t *>(nullptr),
                          static_cast<int64_t>(0), std::max<size_t>(n, 1), rocprim::plus<int64_t>());
  return tb;
}

int sort_pairs(void *tmp, size_t tmp_bytes, const uint64_t *kin, uint64_t *kout, const int32_t *vin, int32_t *vout,
               int64_t n, int end_bit, hipStream_t st) {
  if (n == 0) return SSLA_OK;
  size_t tb = tmp_bytes;
  const hipError_t e = rocprim::radix_sort_pairs<SortConfig>(tmp, tb, kin, kout, vin, vout, static_cast<size_t>(n), 0,
                                                 std::min(std::max(end_bit, 1), 64), st);
  if (e != hipSuccess) {
    set_error("radix sort failed: %s", hipGetErrorString(e));
    return SSLA_ERR_LAUNCH;
  }
  return SSLA_OK;
}

// Exclusive prefix sum of up to kSmallScan values in one workgroup (one
// launch; rocPRIM's scan takes two).  Thread t owns values 8t .. 8t+7; the
// thread totals are scanned across each wavefront with shuffles and across
// the 16 wavefronts through LDS.  Every value is read before any is
// written, so in == out is allowed.  total (optional) receives the sum.
constexpr int kScanThreads = 1024, kScanPer = 8;
constexpr int64_t kSmallScan = static_cast<int64_t>(kScanThreads) * kScanPer;

// Scan inputs: an array, or the segment-head flag of a pooling plan's
// field rows computed on the fly (and stored to head): 1 where row r
// starts a segment -- the first row, a new field, or a time different from
// the row before (reference sparse_pooling.py:26-31) -- 0 at rows past the
// row count *n_rows (read on the device).
struct ArrayIn {
  const int64_t *p;
  __device__ __forceinline__ int64_t operator()(int64_t i) const { return p[i]; }
};
struct RowHeadsIn {
  const int32_t *fidx;
  const int64_t *tim, *n_rows;
  int64_t cap;
  int64_t *head;
  __device__ __forceinline__ int64_t operator()(int64_t r) const {
    const int64_t n = min(*n_rows, cap);
    const int64_t h = (r < n && (r == 0 || fidx[r] != fidx[r - 1] || tim[r] != tim[r - 1])) ? 1 : 0;
    head[r] = h;
    return h;
  }
};

// The sample lengths clamped to [0, N] (group_events' valid rows per
// sample), 0 at i >= B.
struct TruncIn {
  const int64_t *len;
  int64_t B, N;
  __device__ __forceinline__ int64_t operator()(int64_t i) const {
    return i < B ? min(max(len[i], (int64_t)0), N) : 0;
  }
};
// A pixel-sort histogram (int32), each counter cleared as it is read so the
// next pass can count into the same memory.
struct HistIn {
  int32_t *h;
  __device__ __forceinline__ int64_t operator()(int64_t i) const {
    const int64_t v = h[i];
    h[i] = 0;
    return v;
  }
};
// group_events' group-head flag of sorted slot i (first of its pixel; the
// slots at or past E = *Ep are padding), also stored to head.
struct SortedHeadsIn {
  const uint64_t *key;
  const int64_t *Ep;
  int64_t *head;
  __device__ __forceinline__ int64_t operator()(int64_t i) const {
    const int64_t h = (i < *Ep && (i == 0 || key[i] != key[i - 1])) ? 1 : 0;
    head[i] = h;
    return h;
  }
};

template <class In>
__global__ __launch_bounds__(kScanThreads) void small_excl_scan(In in, int64_t *out, int64_t n, int64_t *total) {
  __shared__ int64_t wsum[kScanThreads / 64];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int64_t v[kScanPer];
  int64_t s = 0;
#pragma unroll
  for (int e = 0; e < kScanPer; ++e) {
    const int64_t i = static_cast<int64_t>(t) * kScanPer + e;
    v[e] = i < n ? in(i) : 0;
    s += v[e];
  }
  int64_t x = s;   // inclusive scan of the thread totals across the wavefront
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  int64_t run = x - s;
  for (int j = 0; j < w; ++j) run += wsum[j];
#pragma unroll
  for (int e = 0; e < kScanPer; ++e) {
    const int64_t i = static_cast<int64_t>(t) * kScanPer + e;
    if (i < n) out[i] = run;
    run += v[e];
  }
  if (total && t == kScanThreads - 1) *total = run;
}

// Exclusive prefix sum in one launch for any size: tiles of kLbTile values,
// each tile's workgroup taking its tile index from a ticket (so every tile
// before it is already resident), publishing its aggregate and then its
// inclusive prefix in a flag word per tile, and folding its predecessors'
// words (decoupled look-back: the first wavefront reads 64 flags at a time
// and stops at the nearest inclusive prefix).  The state -- the ticket and
// one flag per tile, lb_state_words(n) words -- must be zero at launch: the
// set-up kernel of each caller clears it.  Flag word: [63:62] state (0 none,
// 1 aggregate, 2 inclusive prefix), [61:0] the value (two's complement), so
// the payload travels with its state and relaxed agent-scope atomics
// suffice.  total (optional) receives the sum.
constexpr int kLbThreads = 1024, kLbPer = 4;
constexpr int64_t kLbTile = static_cast<int64_t>(kLbThreads) * kLbPer;
constexpr uint64_t kLbAgg = 1ull << 62, kLbIncl = 2ull << 62, kLbMask = (1ull << 62) - 1;

inline int64_t lb_state_words(int64_t n) { return 1 + (std::max<int64_t>(n, 1) + kLbTile - 1) / kLbTile; }

__device__ __forceinline__ int64_t lb_value(uint64_t w) { return static_cast<int64_t>(w << 2) >> 2; }

template <class In>
__global__ __launch_bounds__(kLbThreads) void lb_excl_scan(In in, int64_t *__restrict__ out, int64_t n, uint64_t *state,
                                                           int64_t *total) {
  __shared__ int64_t s_tile, s_excl;
  __shared__ int64_t wsum[kLbThreads / 64];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  if (t == 0) s_tile = static_cast<int64_t>(atomicAdd(reinterpret_cast<unsigned long long *>(state), 1ull));
  __syncthreads();
  const int64_t tile = s_tile;
  uint64_t *flags = state + 1;
  const int64_t base = tile * kLbTile + static_cast<int64_t>(t) * kLbPer;
  int64_t v[kLbPer];
  int64_t s = 0;
#pragma unroll
  for (int e = 0; e < kLbPer; ++e) {
    v[e] = base + e < n ? in(base + e) : 0;
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
  if (w == 0) {
    int64_t agg = 0;
    for (int j = 0; j < kLbThreads / 64; ++j) agg += wsum[j];
    int64_t ex = 0;
    if (tile > 0) {
      if (lane == 0)
        __hip_atomic_store(&flags[tile], kLbAgg | (static_cast<uint64_t>(agg) & kLbMask), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      int64_t j_end = tile;   // tiles [0, j_end) not folded yet
      while (true) {
        const int64_t j = j_end - 1 - lane;
        const uint64_t fw = j >= 0 ? __hip_atomic_load(&flags[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : kLbIncl;   // before tile 0: inclusive prefix 0
        const uint64_t st = fw >> 62;
        const uint64_t incl = __builtin_amdgcn_ballot_w64(st == 2);
        const uint64_t none = __builtin_amdgcn_ballot_w64(st == 0);
        const int last = incl ? __builtin_ctzll(incl) : 63;   // lanes [0, last] are needed
        const uint64_t need = last == 63 ? ~0ull : ((2ull << last) - 1);
        if (none & need) {
          __builtin_amdgcn_s_sleep(1);
          continue;
        }
        int64_t val = lane <= last ? lb_value(fw) : 0;
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) val += __shfl_xor(val, d, 64);
        ex += val;
        if (incl) break;
        j_end -= 64;
      }
    }
    if (lane == 0) {
      __hip_atomic_store(&flags[tile], kLbIncl | (static_cast<uint64_t>(ex + agg) & kLbMask), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      s_excl = ex;
      if (total && tile == static_cast<int64_t>(gridDim.x) - 1) *total = ex + agg;
    }
  }
  __syncthreads();
  int64_t run = s_excl + x - s;
  for (int j = 0; j < w; ++j) run += wsum[j];
#pragma unroll
  for (int e = 0; e < kLbPer; ++e) {
    if (base + e < n) out[base + e] = run;
    run += v[e];
  }
}

__global__ void total_from_scan(const int64_t *excl, const int64_t *val, int64_t n, int64_t *dst);

// out = exclusive prefix sum of in[0..n).  Up to kSmallScan values: one
// workgroup.  Above: the one-launch look-back scan when the caller hands a
// zeroed state (lb, lb_state_words(n) words), else rocPRIM's scan.  total
// (optional) receives the sum (0 for n = 0).
// One launch of an exclusive scan of in(0..n) (n > 0): a single workgroup up
// to kSmallScan values, else the look-back scan on the zeroed state lb.
template <class In>
void excl_scan_launch(In in, int64_t *out, int64_t n, uint64_t *lb, int64_t *total, hipStream_t st) {
  if (n <= kSmallScan)
    hipLaunchKernelGGL((small_excl_scan<In>), dim3(1), dim3(kScanThreads), 0, st, in, out, n, total);
  else
    hipLaunchKernelGGL((lb_excl_scan<In>), dim3(static_cast<unsigned>((n + kLbTile - 1) / kLbTile)), dim3(kLbThreads),
                       0, st, in, out, n, lb, total);
}

int excl_scan(void *tmp, size_t tmp_bytes, const int64_t *in, int64_t *out, int64_t n, hipStream_t st,
              uint64_t *lb = nullptr, int64_t *total = nullptr) {
  if (n == 0) {
    if (total) hipLaunchKernelGGL(total_from_scan, dim3(1), dim3(64), 0, st, out, in, (int64_t)0, total);
    return SSLA_OK;
  }
  if (n <= kSmallScan || lb) {
    excl_scan_launch(ArrayIn{in}, out, n, lb, total, st);
    return SSLA_OK;
  }
  size_t tb = tmp_bytes;
  const hipError_t e = rocprim::exclusive_scan(tmp, tb, in, out, static_cast<int64_t>(0), static_cast<size_t>(n),
                                               rocprim::plus<int64_t>(), st);
  if (e != hipSuccess) {
    set_error("prefix sum failed: %s", hipGetErrorString(e));
    return SSLA_ERR_LAUNCH;
  }
  if (total) hipLaunchKernelGGL(total_from_scan, dim3(1), dim3(64), 0, st, out, in, n, total);
  return SSLA_OK;
}

// ------------------------------------------------------------ utilities --
__global__ void fill_i64(int64_t *p, int64_t n, int64_t v) { GRID_STRIDE(i, n) p[i] = v; }
__global__ void fill_i32(int32_t *p, int64_t n, int32_t v) { GRID_STRIDE(i, n) p[i] = v; }
__global__ void iota_i32(int32_t *p, int64_t n) { GRID_STRIDE(i, n) p[i] = static_cast<int32_t>(i); }

// One launch for a call's set-up fills: the 8 count words and 8 status
// flags to zero, a[0..na) = va, b[0..nb) = vb, c[0..nc) = vb, d[0..nd) = vb
// and z[0..nz) = 0 (look-back scan states; any range may be empty).  Grid:
// grid_for(max(8, na, nb, nc, nd, nz)).
__global__ void clear_and_fill(int64_t *counts, int32_t *bad, int64_t *a, int64_t na, int64_t va, int32_t *b,
                               int64_t nb, int32_t vb, int32_t *c, int64_t nc, uint64_t *z = nullptr,
                               int64_t nz = 0, int32_t *d = nullptr, int64_t nd = 0) {
  GRID_STRIDE(i, 8) {
    counts[i] = 0;
    bad[i] = 0;
  }
  GRID_STRIDE(i, na) a[i] = va;
  GRID_STRIDE(i, nb) b[i] = vb;
  GRID_STRIDE(i, nc) c[i] = vb;
  GRID_STRIDE(i, nz) z[i] = 0;
  GRID_STRIDE(i, nd) d[i] = vb;
}

// Sorted-fill set-up in one launch: inv and dst to -1, and the field
// index / length rows of the plan copied to the outputs.
__global__ void rf_sorted_setup(int32_t *inv, int64_t n_inv, int32_t *dst, int64_t n_dst, int64_t *f_index,
                                const int64_t *plan_index, int64_t *f_len, const int64_t *plan_len, int64_t n_act) {
  GRID_STRIDE(i, n_inv) inv[i] = -1;
  GRID_STRIDE(i, n_dst) dst[i] = -1;
  GRID_STRIDE(i, n_act) {
    f_index[i] = plan_index[i];
    f_len[i] = plan_len[i];
  }
}

// counts[k] = a[n-1] + b[n-1] (inclusive total from an exclusive scan), or 0.
__global__ void total_from_scan(const int64_t *excl, const int64_t *val, int64_t n, int64_t *dst) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *dst = n > 0 ? excl[n - 1] + val[n - 1] : 0;
}

// (q, r) = (t / d, t % d): in 32 bits when the kernel's whole index range
// fits (`small`, the same for every thread of a launch) instead of through
// the 64-bit division's emulation
__device__ __forceinline__ void div_index(int64_t t, int d, bool small, int64_t &q, int &r) {
  if (small) {
    const uint32_t t32 = static_cast<uint32_t>(t), qq = t32 / static_cast<uint32_t>(d);
    q = qq;
    r = static_cast<int>(t32 - qq * static_cast<uint32_t>(d));
  } else {
    q = t / d;
    r = static_cast<int>(t - q * d);
  }
}

// out[j, :] = src[idx[j], :] (rows of C floats); idx outside [0, n_src) -> 0.
__global__ void gather_rows_kernel(const float *__restrict__ src, const int64_t *__restrict__ idx, int64_t m,
                                   int64_t n_src, int C, float *__restrict__ out) {
  const bool small = m * C < 0x7fffffff;
  GRID_STRIDE(t, m * C) {
    int64_t j;
    int c;
    div_index(t, C, small, j, c);
    const int64_t r = idx[j];
    out[t] = (r >= 0 && r < n_src) ? src[r * C + c] : 0.f;
  }
}

// out[i] = val[segment of i] for segments given by exclusive offsets `start`
// (n_seg segments over n elements); one thread per segment.
__global__ void expand_segments(const int64_t *__restrict__ val, const int64_t *__restrict__ start,
                                const int64_t *__restrict__ len, int64_t n_seg, int64_t n, int64_t *__restrict__ out) {
  GRID_STRIDE(s, n_seg) {
    const int64_t b = min(max(start[s], (int64_t)0), n), e = min(b + max(len[s], (int64_t)0), n);
    for (int64_t i = b; i < e; ++i) out[i] = val[s];
  }
}

// ------------------------------------------------------------- grouping --
// Per padded slot (b, j < lengths[b]): the flat event index f = off[b] + j,
// the pixel id (formed in fp32 as the reference does, exact below 2^24) and
// the padded row of f.
// Keys of the valid events at their compacted slots f = off[b] + j and the
// padding slots [E, cap) (E = off[B]: key n_pix, sorting last; val = the
// slot, row 0); each slot is written by one thread.  hist (optional): the
// first pass of the pixel sort counts every slot's low digit (key &
// (2^d1 - 1)) in its tile (slot / kRsTile), hist[digit * n_tiles + tile].
constexpr int kRsSteps = 16, kRsTile = 64 * kRsSteps;
__global__ void ge_keys(const float *__restrict__ ev, const int64_t *__restrict__ lengths,
                        const int64_t *__restrict__ off, int B, int64_t N, int C, int H, int W,
                        uint64_t *__restrict__ key, int32_t *__restrict__ val, int64_t *__restrict__ row_of,
                        int32_t *__restrict__ bad, int32_t *__restrict__ hist, int d1, int64_t n_tiles) {
  const int64_t E = off[B];
  const uint64_t mask1 = (uint64_t{1} << d1) - 1;
  GRID_STRIDE(s, static_cast<int64_t>(B) * N) {   // B * N < 2^31 (checked by the caller)
    if (s >= E) {
      const uint64_t k = static_cast<uint64_t>(B) * H * W;
      key[s] = k;
      val[s] = static_cast<int32_t>(s);
      row_of[s] = 0;
      if (hist) atomicAdd(&hist[static_cast<int64_t>(k & mask1) * n_tiles + s / kRsTile], 1);
    }
    const uint32_t s32 = static_cast<uint32_t>(s), b32 = s32 / static_cast<uint32_t>(N);
    const int64_t b = b32, j = s32 - b32 * static_cast<uint32_t>(N);
    if (j >= min(max(lengths[b], (int64_t)0), N)) continue;
    const int64_t f = off[b] + j;
    const float x = ev[s * C + 0], y = ev[s * C + 1];
    const float pid = static_cast<float>(b * static_cast<int64_t>(H) * W) + y * static_cast<float>(W) + x;
    if (!(x >= 0.f && x < W && y >= 0.f && y < H)) *bad = 1;
    // out-of-frame events (reported through bad) stay inside the sorted bits
    const uint64_t n_pix = static_cast<uint64_t>(B) * H * W;
    const uint64_t k = pid >= 0.f ? min(static_cast<uint64_t>(pid), n_pix) : 0;
    key[f] = k;
    val[f] = static_cast<int32_t>(f);
    row_of[f] = s;
    if (hist) atomicAdd(&hist[static_cast<int64_t>(k & mask1) * n_tiles + f / kRsTile], 1);
  }
}

// One pass of the pixel sort (a stable LSD counting sort): the digit of a
// key is (key >> shift) & (2^d - 1); off[digit * n_tiles + tile] is where
// the tile's keys of that digit start (the exclusive prefix of the pass's
// histogram in digit-major order).  A workgroup per tile of kRsTile slots,
// 16 / S wavefronts each taking S rows of 64 in order.  Within a row the
// lanes with equal digits find each other with one ballot per digit bit and
// rank by lane; the lowest of them adds their count to the wavefront's LDS
// counter of the digit (so a lane's rank within its wavefront is that
// counter's old value plus the lanes below it with its digit).  The
// counters are then turned into per-digit prefixes over the wavefronts, so
// a key's place is the digit's start + the keys of that digit in earlier
// wavefronts + its rank: slot order within the tile, equal keys keep their
// order.  FIRST: also counts the next pass's digits (shift2, d2) at the
// destination tiles into hist2.  Destinations outside [0, n) (inconsistent
// counts) are skipped.  LDS: (16 / S + 1) * 2^d int32.
template <bool FIRST, int S>
__global__ __launch_bounds__(64 * (kRsSteps / S)) void rs_scatter(
    const uint64_t *__restrict__ kin, const int32_t *__restrict__ vin, int64_t n, int64_t n_tiles, int shift, int d,
    const int64_t *__restrict__ off, uint64_t *__restrict__ kout, int32_t *__restrict__ vout, int shift2, int d2,
    int32_t *__restrict__ hist2) {
  constexpr int kW = kRsSteps / S;
  extern __shared__ int32_t rs_lds[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t t = blockIdx.x;
  const uint32_t R = 1u << d;
  int32_t *rs_base = rs_lds, *rs_cnt = rs_lds + R;   // rs_cnt[w * R + digit]
  for (uint32_t r = tid; r < R; r += 64 * kW) {
    rs_base[r] = static_cast<int32_t>(off[static_cast<int64_t>(r) * n_tiles + t]);
#pragma unroll
    for (int q = 0; q < kW; ++q) rs_cnt[q * R + r] = 0;
  }
  __syncthreads();
  const int64_t base = t * kRsTile + static_cast<int64_t>(w) * S * 64;
  uint64_t k[S];
  int32_t v[S], rank[S];
  uint32_t dig[S];
#pragma unroll
  for (int st = 0; st < S; ++st) {
    const int64_t i = base + st * 64 + lane;
    k[st] = i < n ? kin[i] : 0;
    v[st] = i < n ? vin[i] : 0;
  }
  const uint64_t below = (uint64_t{1} << lane) - 1;
  int32_t *cnt = rs_cnt + static_cast<int64_t>(w) * R;
#pragma unroll
  for (int st = 0; st < S; ++st) {
    const bool valid = base + st * 64 + lane < n;
    const uint32_t r = static_cast<uint32_t>(k[st] >> shift) & (R - 1);
    uint64_t m = __builtin_amdgcn_ballot_w64(valid);
    for (int b = 0; b < d; ++b) {
      const bool bit = (r >> b) & 1u;
      const uint64_t bal = __builtin_amdgcn_ballot_w64(bit);
      m &= bit ? bal : ~bal;
    }
    const int leader = valid ? __builtin_ctzll(m) : lane;
    int32_t old = 0;
    if (valid && lane == leader) {
      old = cnt[r];
      cnt[r] = old + __builtin_popcountll(m);
    }
    old = __shfl(old, leader, 64);
    rank[st] = old + __builtin_popcountll(m & below);
    dig[st] = r;
  }
  __syncthreads();
  // per digit: the counts of the wavefronts before each one
  for (uint32_t r = tid; r < R; r += 64 * kW) {
    int32_t run = 0;
#pragma unroll
    for (int q = 0; q < kW; ++q) {
      const int32_t c = rs_cnt[q * R + r];
      rs_cnt[q * R + r] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int st = 0; st < S; ++st) {
    if (base + st * 64 + lane >= n) continue;
    const uint32_t r = dig[st];
    const int64_t pos = static_cast<int64_t>(rs_base[r]) + cnt[r] + rank[st];
    if (pos < 0 || pos >= n) continue;
    kout[pos] = k[st];
    vout[pos] = v[st];
    if constexpr (FIRST) {
      const uint32_t r2 = static_cast<uint32_t>(k[st] >> shift2) & ((1u << d2) - 1);
      atomicAdd(&hist2[static_cast<int64_t>(r2) * n_tiles + pos / kRsTile], 1);
    }
  }
}

// A pass of the pixel sort with the widest wavefront split whose counters
// stay within 50 KB of LDS (S rows per wavefront: 1 up to 2^9 digits, 2 at
// 2^10, 4 at 2^11, 8 at 2^12).
template <bool FIRST>
void rs_pass(const uint64_t *kin, const int32_t *vin, int64_t n, int64_t n_tiles, int shift, int d,
             const int64_t *off, uint64_t *kout, int32_t *vout, int shift2, int d2, int32_t *hist2, hipStream_t st) {
  const unsigned tiles = static_cast<unsigned>(n_tiles);
  const int S = d <= 9 ? 1 : (d == 10 ? 2 : (d == 11 ? 4 : 8));
  const size_t lds = (static_cast<size_t>(kRsSteps / S) + 1) * (size_t{1} << d) * sizeof(int32_t);
  if (S == 1)
    hipLaunchKernelGGL((rs_scatter<FIRST, 1>), dim3(tiles), dim3(64 * kRsSteps), lds, st, kin, vin, n, n_tiles, shift,
                       d, off, kout, vout, shift2, d2, hist2);
  else if (S == 2)
    hipLaunchKernelGGL((rs_scatter<FIRST, 2>), dim3(tiles), dim3(64 * kRsSteps / 2), lds, st, kin, vin, n, n_tiles,
                       shift, d, off, kout, vout, shift2, d2, hist2);
  else if (S == 4)
    hipLaunchKernelGGL((rs_scatter<FIRST, 4>), dim3(tiles), dim3(64 * kRsSteps / 4), lds, st, kin, vin, n, n_tiles,
                       shift, d, off, kout, vout, shift2, d2, hist2);
  else
    hipLaunchKernelGGL((rs_scatter<FIRST, 8>), dim3(tiles), dim3(64 * kRsSteps / 8), lds, st, kin, vin, n, n_tiles,
                       shift, d, off, kout, vout, shift2, d2, hist2);
}

// group starts and the group count (counts[0] = G); start[G] = E
__global__ void ge_starts(const int64_t *__restrict__ head, const int64_t *__restrict__ gpos, int64_t cap,
                          const int64_t *__restrict__ Ep, int64_t *__restrict__ start, int64_t *__restrict__ counts) {
  const int64_t E = *Ep;
  GRID_STRIDE(i, cap) {
    if (i < E && head[i]) start[gpos[i]] = i;
    if (i == 0) {
      const int64_t G = E > 0 ? gpos[E - 1] + head[E - 1] : 0;
      counts[0] = G;
      start[G] = E;
    }
  }
}

// per group: kept length and the group's pixel attributes (kept = 0 beyond G)
// kept[g]: the group's latest cap_px events, of which the first keep_first
// stay (keep_first = INT64_MAX: all of them).
__global__ void ge_groups(const int64_t *__restrict__ counts, const int64_t *__restrict__ start, int64_t cap,
                          const int32_t *__restrict__ order, const int64_t *__restrict__ row_of,
                          const float *__restrict__ ev, int64_t N, int C, int cap_px, int64_t keep_first,
                          int64_t *__restrict__ kept, int64_t *__restrict__ gr_batch, int64_t *__restrict__ gr_h,
                          int64_t *__restrict__ gr_w, int64_t *__restrict__ gr_len) {
  const int64_t G = counts[0];
  GRID_STRIDE(g, cap) {
    if (g >= G) {
      kept[g] = 0;
      continue;
    }
    const int64_t s = start[g], e = start[g + 1];
    const int64_t k = min(min(e - s, static_cast<int64_t>(cap_px)), keep_first);
    kept[g] = k;
    gr_len[g] = k;
    const int64_t r = row_of[order[s]];
    gr_batch[g] = r / N;
    gr_w[g] = static_cast<int64_t>(ev[r * C + 0]);
    gr_h[g] = static_cast<int64_t>(ev[r * C + 1]);
  }
}

// Emit the kept events of every group (its latest cap_px, then the first
// kept[g] of those): features are columns fc .. C-1.  DELAYS: column fc (a
// timestamp) becomes the delay since the group's previous event, (t - t')
// / 1e5 in fp32 capped at 1, and 1 for the first of the latest cap_px
// (MosModel.preprocess_inputs, model_mos.py:194-201).
template <bool DELAYS>
__global__ void ge_emit(const int64_t *__restrict__ head, const int64_t *__restrict__ gpos,
                        const int64_t *__restrict__ start, const int64_t *__restrict__ kept,
                        const int64_t *__restrict__ kpre, const int32_t *__restrict__ order,
                        const int64_t *__restrict__ row_of, const float *__restrict__ ev, int64_t cap,
                        const int64_t *__restrict__ Ep, int C, int cap_px, int fc, float *__restrict__ out_ev,
                        int64_t *__restrict__ out_t) {
  const int64_t E = *Ep;
  const int F = C - fc;
  GRID_STRIDE(i, cap) {
    if (i >= E) continue;
    const int64_t g = gpos[i] + head[i] - 1;
    const int64_t s = start[g], e = start[g + 1];
    const int64_t drop = (e - s) - min(e - s, static_cast<int64_t>(cap_px));
    const int64_t rank = i - s - drop;
    if (rank < 0 || rank >= kept[g]) continue;
    const int64_t o = kpre[g] + rank;
    const int64_t r = row_of[order[i]];
    const float *src = ev + r * C;
    for (int c = fc; c < C; ++c) out_ev[o * F + (c - fc)] = src[c];
    if constexpr (DELAYS) {
      float d = 1.f;
      if (rank > 0) d = fminf((src[fc] - ev[row_of[order[i - 1]] * C + fc]) / 1e5f, 1.f);
      out_ev[o * F] = d;
    }
    out_t[o] = static_cast<int64_t>(src[2]);
  }
}

// ----------------------------------------------------------------- LUTs --
__global__ void lut_kernel(int H, int W, int kh, int kw, int sh, int sw, int top, int left, int Ho, int Wo,
                           int64_t *__restrict__ lut, int64_t *__restrict__ outc) {
  const int64_t n = static_cast<int64_t>(Ho) * Wo * kh * kw;
  GRID_STRIDE(t, n) {
    const int64_t rf = t / (kh * kw), a = t % (kh * kw);
    const int oy = static_cast<int>(rf / Wo), ox = static_cast<int>(rf % Wo);
    const int y = oy * sh - top + static_cast<int>(a / kw), x = ox * sw - left + static_cast<int>(a % kw);
    lut[t] = (y >= 0 && y < H && x >= 0 && x < W) ? static_cast<int64_t>(y) * W + x : -1;
    if (outc && a == 0) {
      outc[2 * rf] = ox;
      outc[2 * rf + 1] = oy;
    }
  }
}

// ---------------------------------------------------- field / patch scatter --
// pixel map: pixmap[b*H*W + h*W + w] = group index
// (inv non-null: also inv[p * A + a] = rf with lut[rf * A + a] == p, the
// inverse table of the counting fill, in the same launch; with one_field,
// for layouts where every pixel lies in at most one field, inv[p] = rf * A
// + a instead, and *overlap = 1 if a pixel turns out to lie in two)
__global__ void rf_pixmap(const int64_t *__restrict__ gb, const int64_t *__restrict__ gh,
                          const int64_t *__restrict__ gw, int64_t G, int H, int W, int64_t n_pix,
                          int32_t *__restrict__ pixmap, int32_t *__restrict__ bad, const int64_t *__restrict__ lut,
                          int64_t n_rf, int A, int32_t *__restrict__ inv, int one_field,
                          int64_t *__restrict__ overlap) {
  GRID_STRIDE(g, G) {
    const int64_t p = gb[g] * H * W + gh[g] * W + gw[g];
    if (gh[g] < 0 || gh[g] >= H || gw[g] < 0 || gw[g] >= W || p < 0 || p >= n_pix) {
      *bad = 1;
      continue;
    }
    pixmap[p] = static_cast<int32_t>(g);
  }
  if (inv) {
    const int64_t HW = static_cast<int64_t>(H) * W;
    GRID_STRIDE(t, n_rf * A) {
      const int64_t p = lut[t];
      if (p >= 0 && p < HW) {
        if (one_field) {   // a second field at the same pixel breaks the promise: reported
          if (atomicCAS(&inv[p], -1, static_cast<int32_t>(t)) != -1) *overlap = 1;
        } else {
          inv[p * A + t % A] = static_cast<int32_t>(t / A);
        }
      }
    }
  }
}

// per field (b, rf): number of events, active flag, and (pk non-null) both
// packed as nev * 2^21 + act, so that one prefix sum yields both
constexpr int kPackBits = 21;
__global__ void rf_count(const int64_t *__restrict__ lut, int64_t n_rf, int A, int B, int H, int W,
                         const int32_t *__restrict__ pixmap, const int64_t *__restrict__ glen,
                         int64_t *__restrict__ nev, int64_t *__restrict__ act, int64_t *__restrict__ pk) {
  GRID_STRIDE(f, static_cast<int64_t>(B) * n_rf) {
    const int64_t b = f / n_rf, r = f % n_rf;
    int64_t n = 0, a_ = 0;
    for (int a = 0; a < A; ++a) {
      const int64_t p = lut[r * A + a];
      if (p < 0) continue;
      const int32_t g = pixmap[b * H * W + p];
      if (g < 0) continue;
      a_ = 1;
      n += glen[g];
    }
    nev[f] = n;
    act[f] = a_;
    if (pk) pk[f] = (n << kPackBits) | a_;
  }
}

// rf_count with one lane per (field, kernel position) when A divides 64:
// the A lanes of a field sit in one wavefront and sum their events with
// shuffles, so each lane makes one lookup chain instead of A in a row.
// Grid: exactly ceil(B * n_rf * A / kThreads) workgroups (every lane takes
// part in the shuffles; lanes past the end add nothing and write nothing).
__global__ void rf_count_lanes(const int64_t *__restrict__ lut, int64_t n_rf, int A, int B, int H, int W,
                               const int32_t *__restrict__ pixmap, const int64_t *__restrict__ glen,
                               int64_t *__restrict__ nev, int64_t *__restrict__ act, int64_t *__restrict__ pk) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t n_f = static_cast<int64_t>(B) * n_rf;
  const int64_t f = t / A;
  const int a = static_cast<int>(t - f * A);
  int64_t n = 0, on = 0;
  if (f < n_f) {
    const int64_t b = f / n_rf, r = f - b * n_rf;
    const int64_t p = lut[r * A + a];
    const int32_t g = p >= 0 ? pixmap[b * H * W + p] : -1;
    if (g >= 0) {
      n = glen[g];
      on = 1;
    }
  }
  for (int d = 1; d < A; d <<= 1) {
    n += __shfl_xor(n, d, 64);
    on |= __shfl_xor(on, d, 64);
  }
  if (f < n_f && a == 0) {
    nev[f] = n;
    act[f] = on;
    if (pk) pk[f] = (n << kPackBits) | on;
  }
}

// From the prefix sum of the packed pairs, in one launch: act_pre / ev_pre
// of every field, the flat index and event count of every active field
// (f_index / f_len at its active index, as rf_fields writes them) and the
// totals (counts[0], counts[1]).
__global__ void rf_unpack_fields(const int64_t *__restrict__ pk_pre, const int64_t *__restrict__ pk, int64_t n,
                                 int64_t *__restrict__ act_pre, int64_t *__restrict__ ev_pre,
                                 int64_t *__restrict__ counts, int64_t *__restrict__ f_index,
                                 int64_t *__restrict__ f_len) {
  constexpr int64_t mask = (int64_t{1} << kPackBits) - 1;
  GRID_STRIDE(f, n) {
    const int64_t pre = pk_pre[f], v = pk[f];
    act_pre[f] = pre & mask;
    ev_pre[f] = pre >> kPackBits;
    if (v & mask) {
      f_index[pre & mask] = f;
      f_len[pre & mask] = v >> kPackBits;
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const int64_t t = n > 0 ? pk_pre[n - 1] + pk[n - 1] : 0;
    counts[0] = t & mask;
    counts[1] = t >> kPackBits;
  }
}

// enumerate the events of every active field (pixels in kernel-coordinate
// order, each pixel's run in group order): sort key, source event, position
__global__ void rf_enumerate(const int64_t *__restrict__ lut, int64_t n_rf, int A, int B, int H, int W,
                             const int32_t *__restrict__ pixmap, const int64_t *__restrict__ glen,
                             const int64_t *__restrict__ gstart, const int64_t *__restrict__ act,
                             const int64_t *__restrict__ act_pre, const int64_t *__restrict__ ev_pre,
                             const int64_t *__restrict__ time, int64_t E_in, uint64_t t_stride,
                             uint64_t *__restrict__ key, int32_t *__restrict__ val, int64_t *__restrict__ pre_src,
                             int64_t *__restrict__ pre_pos) {
  GRID_STRIDE(t, static_cast<int64_t>(B) * n_rf * A) {
    const int64_t f = t / A;
    const int a = static_cast<int>(t % A);
    if (!act[f]) continue;
    const int64_t b = f / n_rf, r = f % n_rf;
    const int64_t p = lut[r * A + a];
    if (p < 0) continue;
    const int32_t g = pixmap[b * H * W + p];
    if (g < 0) continue;
    int64_t o = ev_pre[f];
    for (int a2 = 0; a2 < a; ++a2) {
      const int64_t p2 = lut[r * A + a2];
      if (p2 < 0) continue;
      const int32_t g2 = pixmap[b * H * W + p2];
      if (g2 >= 0) o += glen[g2];
    }
    const uint64_t fk = static_cast<uint64_t>(act_pre[f]) * t_stride;
    const int64_t s = gstart[g];
    for (int64_t e = 0; e < glen[g]; ++e) {
      const int64_t src = min(max(s + e, (int64_t)0), E_in - 1);
      key[o + e] = fk + static_cast<uint64_t>(max(time[src], (int64_t)0));
      val[o + e] = static_cast<int32_t>(o + e);
      pre_src[o + e] = src;
      pre_pos[o + e] = a;
    }
  }
}

// per active field: flat (b, rf) index, event count
__global__ void rf_fields(const int64_t *__restrict__ act, const int64_t *__restrict__ act_pre,
                          const int64_t *__restrict__ nev, int64_t n_f, int64_t *__restrict__ f_index,
                          int64_t *__restrict__ f_len) {
  GRID_STRIDE(f, n_f) {
    if (!act[f]) continue;
    f_index[act_pre[f]] = f;
    f_len[act_pre[f]] = nev[f];
  }
}

// rf_count_lanes, the prefix sum of the packed pairs and rf_unpack_fields
// in one launch (A divides 64; the packed path): workgroups take tickets in
// field order, count their 256 / A fields (one lane per (field, position),
// sums by shuffles), publish the packed total of their fields and find the
// total before them by decoupled look-back (lb_excl_scan's flag words, whose
// state the plan's set-up kernel clears), then write every field's act_pre /
// ev_pre and the compacted index and count of its active fields; the last
// workgroup writes the totals (counts[0], counts[1]).
__global__ __launch_bounds__(256) void rf_count_scan(const int64_t *__restrict__ lut, int64_t n_rf, int A, int B,
                                                     int H, int W, const int32_t *__restrict__ pixmap,
                                                     const int64_t *__restrict__ glen, int64_t *__restrict__ nev,
                                                     int64_t *__restrict__ act, int64_t *__restrict__ act_pre,
                                                     int64_t *__restrict__ ev_pre, int64_t *__restrict__ f_index,
                                                     int64_t *__restrict__ f_len, int64_t *__restrict__ counts,
                                                     uint64_t *state) {
  constexpr int64_t mask = (int64_t{1} << kPackBits) - 1;
  __shared__ int64_t s_tile, s_excl;
  __shared__ int64_t s_pk[256];   // packed pair of each of the workgroup's fields
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid == 0) s_tile = static_cast<int64_t>(atomicAdd(reinterpret_cast<unsigned long long *>(state), 1ull));
  __syncthreads();
  const int64_t tile = s_tile;
  uint64_t *flags = state + 1;
  const int fpw = 256 / A;   // fields per workgroup
  const int64_t n_f = static_cast<int64_t>(B) * n_rf;
  const int64_t t = tile * 256 + tid;
  const int64_t f = t / A;
  const int a = static_cast<int>(t - f * A);
  int64_t n = 0, on = 0;
  if (f < n_f) {
    const int64_t b = f / n_rf, r = f - b * n_rf;
    const int64_t p = lut[r * A + a];
    const int32_t g = p >= 0 ? pixmap[b * H * W + p] : -1;
    if (g >= 0) {
      n = glen[g];
      on = 1;
    }
  }
  for (int d = 1; d < A; d <<= 1) {
    n += __shfl_xor(n, d, 64);
    on |= __shfl_xor(on, d, 64);
  }
  const int fi = tid / A;   // field of this lane within the workgroup
  if (a == 0) s_pk[fi] = f < n_f ? (n << kPackBits) | on : 0;
  __syncthreads();
  if (tid < 64) {
    // exclusive prefix of the workgroup's fields (fpw <= 256: four per lane)
    int64_t v[4], sum = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = 4 * lane + u;
      v[u] = i < fpw ? s_pk[i] : 0;
      sum += v[u];
    }
    int64_t x = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    const int64_t agg = __shfl(x, 63, 64);
    int64_t run = x - sum;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = 4 * lane + u;
      if (i < fpw) s_pk[i] = run;   // now the exclusive prefix within the workgroup
      run += v[u];
    }
    int64_t ex = 0;
    if (tile > 0) {
      if (lane == 0)
        __hip_atomic_store(&flags[tile], kLbAgg | (static_cast<uint64_t>(agg) & kLbMask), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      int64_t j_end = tile;
      while (true) {
        const int64_t j = j_end - 1 - lane;
        const uint64_t fw = j >= 0 ? __hip_atomic_load(&flags[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : kLbIncl;
        const uint64_t st = fw >> 62;
        const uint64_t incl = __builtin_amdgcn_ballot_w64(st == 2);
        const uint64_t none = __builtin_amdgcn_ballot_w64(st == 0);
        const int last = incl ? __builtin_ctzll(incl) : 63;
        const uint64_t need = last == 63 ? ~0ull : ((2ull << last) - 1);
        if (none & need) {
          __builtin_amdgcn_s_sleep(1);
          continue;
        }
        int64_t val = lane <= last ? lb_value(fw) : 0;
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) val += __shfl_xor(val, d, 64);
        ex += val;
        if (incl) break;
        j_end -= 64;
      }
    }
    if (lane == 0) {
      __hip_atomic_store(&flags[tile], kLbIncl | (static_cast<uint64_t>(ex + agg) & kLbMask), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      s_excl = ex;
      if (tile == static_cast<int64_t>(gridDim.x) - 1) {
        counts[0] = (ex + agg) & mask;
        counts[1] = (ex + agg) >> kPackBits;
      }
    }
  }
  __syncthreads();
  if (a == 0 && f < n_f) {
    const int64_t pre = s_excl + s_pk[fi];
    nev[f] = n;
    act[f] = on;
    act_pre[f] = pre & mask;
    ev_pre[f] = pre >> kPackBits;
    if (on) {
      f_index[pre & mask] = f;
      f_len[pre & mask] = n;
    }
  }
}

// o_fidx (optional): the active-field index of every row, the high part of
// its sorted key (active index * t_stride + time).
__global__ void rf_emit(const int32_t *__restrict__ perm, int64_t E_out, const int64_t *__restrict__ pre_src,
                        const int64_t *__restrict__ pre_pos, const int64_t *__restrict__ time,
                        int64_t *__restrict__ o_src, int64_t *__restrict__ o_time, int64_t *__restrict__ o_pos,
                        const uint64_t *__restrict__ skey, uint64_t t_stride, int32_t *__restrict__ o_fidx) {
  GRID_STRIDE(i, E_out) {
    const int32_t k = perm[i];
    const int64_t s = pre_src[k];
    o_src[i] = s;
    if (o_time) o_time[i] = time[s];
    if (o_pos) o_pos[i] = pre_pos[k];
    if (o_fidx) o_fidx[i] = static_cast<int32_t>(skey[i] / t_stride);
  }
}

__global__ void max_i64(const int64_t *__restrict__ x, int64_t n, unsigned long long *__restrict__ dst) {
  __shared__ long long s[kThreads];
  long long m = 0;
  GRID_STRIDE(i, n) m = max(m, static_cast<long long>(x[i]));
  s[threadIdx.x] = m;
  __syncthreads();
  for (int d = kThreads / 2; d > 0; d >>= 1) {
    if (threadIdx.x < d) s[threadIdx.x] = max(s[threadIdx.x], s[threadIdx.x + d]);
    __syncthreads();
  }
  if (threadIdx.x == 0 && s[0] > 0) atomicMax(dst, static_cast<unsigned long long>(s[0]));
}

// ------------------------------------------------------- ordered index add --
// out[r, :] = sum over sorted copies of src rows, in copy order (fp32,
// starting from zero) -- the arithmetic of a sequential index_add_ into zeros.
__global__ void index_add_rows(const float *__restrict__ src, const uint64_t *__restrict__ skey,
                               const int32_t *__restrict__ perm, int64_t n, int64_t n_out, int C,
                               float *__restrict__ out) {
  // one wavefront per output row; binary search of its run in the sorted keys
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (r >= n_out) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (skey[mid] < static_cast<uint64_t>(r)) lo = mid + 1; else hi = mid;
  }
  int64_t e = lo;
  {
    int64_t l2 = lo, h2 = n;
    while (l2 < h2) {
      const int64_t mid = (l2 + h2) >> 1;
      if (skey[mid] <= static_cast<uint64_t>(r)) l2 = mid + 1; else h2 = mid;
    }
    e = l2;
  }
  for (int c0 = 0; c0 < C; c0 += 64) {
    const int c = c0 + lane;
    if (c >= C) continue;
    float acc = 0.f;
    for (int64_t j = lo; j < e; ++j) acc += src[static_cast<int64_t>(perm[j]) * C + c];
    out[r * C + c] = acc;
  }
}

__global__ void idx_keys(const int64_t *__restrict__ idx, int64_t n, int64_t n_out, uint64_t *__restrict__ key,
                         int32_t *__restrict__ val, int32_t *__restrict__ bad) {
  GRID_STRIDE(i, n) {
    const int64_t r = idx[i];
    if (r < 0 || r >= n_out) *bad = 1;
    key[i] = (r >= 0 && r < n_out) ? static_cast<uint64_t>(r) : static_cast<uint64_t>(n_out);
    val[i] = static_cast<int32_t>(i);
  }
}

// ---------------------------------------------------------- truncation --
// keep the first `thr` elements of every sequence
__global__ void trunc_len(const int64_t *__restrict__ len, int64_t n, int64_t thr, int64_t *__restrict__ kl) {
  GRID_STRIDE(s, n) kl[s] = min(max(len[s], (int64_t)0), thr);
}
__global__ void trunc_copy(const float *__restrict__ data, const int64_t *__restrict__ others,
                           const int64_t *__restrict__ start, const int64_t *__restrict__ kl,
                           const int64_t *__restrict__ kpre, int64_t n_seq, int64_t E, int C,
                           float *__restrict__ out, int64_t *__restrict__ out_o) {
  GRID_STRIDE(s, n_seq) {
    for (int64_t j = 0; j < kl[s]; ++j) {
      const int64_t src = min(start[s] + j, E - 1), dst = kpre[s] + j;
      for (int c = 0; c < C; ++c) out[dst * C + c] = data[src * C + c];
      if (others) out_o[dst] = others[src];
    }
  }
}

// ------------------------------------------------------ temporal dropout --
__global__ void td_len(const int64_t *__restrict__ len, int64_t n, int64_t w, int64_t *__restrict__ kl) {
  GRID_STRIDE(s, n) kl[s] = (max(len[s], (int64_t)0) + w - 1) / w;
}
__global__ void td_index(const int64_t *__restrict__ len, const int64_t *__restrict__ start,
                         const int64_t *__restrict__ kl, const int64_t *__restrict__ kpre, int64_t n, int64_t w,
                         int64_t cap, int64_t *__restrict__ idx) {
  GRID_STRIDE(s, n) {
    const int64_t L = max(len[s], (int64_t)0);
    const int64_t off = ((L % w - 1) % w + w) % w;
    const int64_t end = min(kpre[s] + kl[s], cap);   // rows past the capacity are counted, not written
    for (int64_t j = kpre[s]; j < end; ++j) idx[j] = start[s] + off + (j - kpre[s]) * w;
  }
}

// --------------------------------------------------------------- pooling --
// key = time + field * (max_t + 1) over fields in order; segment heads
__global__ void pool_heads(const int64_t *__restrict__ time, const int64_t *__restrict__ field, int64_t E,
                           int64_t *__restrict__ head) {
  GRID_STRIDE(i, E) head[i] = (i == 0 || field[i] != field[i - 1] || time[i] != time[i - 1]) ? 1 : 0;
}
__global__ void pool_emit(const int64_t *__restrict__ head, const int64_t *__restrict__ spre,
                          const int64_t *__restrict__ time, const int64_t *__restrict__ field, int64_t E,
                          int64_t *__restrict__ seg, int64_t *__restrict__ seg_time, int64_t *__restrict__ seg_field) {
  GRID_STRIDE(i, E) {
    const int64_t s = spre[i] + head[i] - 1;
    seg[i] = s;
    if (head[i]) {
      seg_time[s] = time[i];
      seg_field[s] = field[i];
    }
  }
}
// The last index j in [0, n) with a[j] <= x, for a non-decreasing a
// (0 when a[0] > x).
__device__ __forceinline__ int64_t last_le(const int64_t *__restrict__ a, int64_t n, int64_t x) {
  int64_t lo = 0, hi = n - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (a[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// The first index j in [0, n) with a[j] >= x (n if none), a non-decreasing.
__device__ __forceinline__ int64_t first_ge(const int64_t *__restrict__ a, int64_t n, int64_t x) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (a[mid] < x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// out[f] = the number of the counts[which] labels equal to f, for labels
// that are non-decreasing (the segments' fields): two binary searches per
// label value, no atomics.
__global__ void count_sorted_by(const int64_t *__restrict__ lab, const int64_t *__restrict__ counts, int which,
                                int64_t n_lab, int64_t *__restrict__ out) {
  const int64_t n = counts[which];
  GRID_STRIDE(f, n_lab) out[f] = first_ge(lab, n, f + 1) - first_ge(lab, n, f);
}

// field[i] = f for the events of field f (fields laid out in order: start
// is the exclusive prefix of the lengths), one thread per event.
__global__ void pool_field_of(const int64_t *__restrict__ start, const int64_t *__restrict__ len, int64_t n_f,
                              int64_t E, int64_t *__restrict__ field) {
  GRID_STRIDE(i, E) {
    const int64_t f = last_le(start, n_f, i);
    if (i >= start[f] && i < start[f] + len[f]) field[i] = f;
  }
}

__global__ void seg_ends(const int64_t *__restrict__ start, const int64_t *__restrict__ len, int64_t n,
                         int64_t *__restrict__ end) {
  GRID_STRIDE(i, n) end[i] = start[i] + len[i];
}

__global__ void store_u64_as_i64(const unsigned long long *__restrict__ src, int64_t *__restrict__ dst) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *dst = static_cast<int64_t>(*src);
}

// ---------------------------------------------------------------- delays --
// column 0 of feat [E, C] holds timestamps; replace them by the per-pixel
// delay (t_i - t_{i-1}) / 1e5 clamped at 1, with 1 for the first event of
// every group (model_mos.py:195-201, fp32 arithmetic as there)
__global__ void pixel_delays(float *__restrict__ feat, const int64_t *__restrict__ start,
                             const int64_t *__restrict__ len, int64_t G, int64_t E, int C) {
  GRID_STRIDE(g, G) {
    const int64_t b = min(max(start[g], (int64_t)0), E), e = min(b + max(len[g], (int64_t)0), E);
    float prev = b > 0 ? feat[(b - 1) * C] : 0.f;
    for (int64_t i = b; i < e; ++i) {
      const float t = feat[i * C];
      feat[i * C] = (i == b) ? 1.f : fminf((t - prev) / 1e5f, 1.f);
      prev = t;
    }
  }
}

// ---------------------------------------------------------------- grids --
// last event of every group at its (b, h, w) cell of a [B, C, Hg, Wg] grid
__global__ void grid_place(const float *__restrict__ ev, const int64_t *__restrict__ gend, const int64_t *__restrict__ gb,
                           const int64_t *__restrict__ gh, const int64_t *__restrict__ gw, int64_t G, int64_t E, int C,
                           int B, int Hg, int Wg, float *__restrict__ grid, int32_t *__restrict__ bad) {
  const bool small = G * C < 0x7fffffff;
  GRID_STRIDE(t, G * C) {
    int64_t g;
    int c;
    div_index(t, C, small, g, c);
    const int64_t b = gb[g], h = gh[g], w = gw[g];
    const int64_t last = gend[g] - 1;
    if (b < 0 || b >= B || h < 0 || h >= Hg || w < 0 || w >= Wg || last < 0 || last >= E) {
      *bad = 1;
      continue;
    }
    // one group per cell, so the reference's index_add_ into zeros is a store
    grid[((b * C + c) * Hg + h) * Wg + w] = ev[last * C + c];
  }
}

// Several grids in one launch: one workgroup per (level, block of kGridCB
// channels).  Each workgroup builds its level's cell -> last-event map in
// LDS from the group lengths (kGridPer groups per thread, a running prefix
// over chunks of kGridThreads * kGridPer groups), then writes its channel
// planes cell by cell, 0 where no group sits: every element is written
// once, so the grid needs no clearing and no two workgroups touch the same
// address.  Loads are issued kGridPer at a time ahead of their uses.
constexpr int kGridThreads = 1024, kGridPer = 4, kGridCB = 4;
struct GridArgs {
  ssla_grid_level lv[SSLA_GRIDS_MAX_LEVELS];
  int blk0[SSLA_GRIDS_MAX_LEVELS + 1];
  int n_levels, B;
};

__global__ __launch_bounds__(kGridThreads) void grids_kernel(GridArgs a, int32_t *status) {
  extern __shared__ int32_t cell_ev[];
  __shared__ int64_t wsum[kGridThreads / 64];
  int L = 0;
  while (L + 1 < a.n_levels && static_cast<int>(blockIdx.x) >= a.blk0[L + 1]) ++L;
  const ssla_grid_level &lv = a.lv[L];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t HW = static_cast<int64_t>(lv.Hg) * lv.Wg, cells = a.B * HW;
  for (int64_t i = tid; i < cells; i += kGridThreads) cell_ev[i] = -1;
  __syncthreads();
  bool bad = false;
  int64_t carry = 0;
  for (int64_t base = 0; base < lv.G; base += kGridThreads * kGridPer) {
    const int64_t g0 = base + static_cast<int64_t>(tid) * kGridPer;
    int64_t len[kGridPer], gb[kGridPer], gh[kGridPer], gw[kGridPer];
    int64_t s = 0;
#pragma unroll
    for (int u = 0; u < kGridPer; ++u) {
      const bool in = g0 + u < lv.G;
      len[u] = in ? lv.lengths[g0 + u] : 0;
      gb[u] = in ? lv.batch[g0 + u] : 0;
      gh[u] = in ? lv.h[g0 + u] : 0;
      gw[u] = in ? lv.w[g0 + u] : 0;
      s += len[u];
    }
    int64_t x = s;   // inclusive scan of the thread sums across the wavefront
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    if (lane == 63) wsum[wv] = x;
    __syncthreads();
    int64_t pre = 0, tot = 0;
#pragma unroll
    for (int j = 0; j < kGridThreads / 64; ++j) {
      pre += j < wv ? wsum[j] : 0;
      tot += wsum[j];
    }
    int64_t end = carry + pre + x - s;
#pragma unroll
    for (int u = 0; u < kGridPer; ++u) {
      end += len[u];
      if (g0 + u >= lv.G) continue;
      const int64_t last = end - 1;
      if (gb[u] < 0 || gb[u] >= a.B || gh[u] < 0 || gh[u] >= lv.Hg || gw[u] < 0 || gw[u] >= lv.Wg || last < 0 ||
          last >= lv.E)
        bad = true;
      else
        cell_ev[(gb[u] * lv.Hg + gh[u]) * lv.Wg + gw[u]] = static_cast<int32_t>(last);
    }
    carry += tot;
    __syncthreads();   // wsum is rewritten by the next chunk
  }
  // (the loop's last barrier orders the map's writes before the reads)
  const int c0 = (static_cast<int>(blockIdx.x) - a.blk0[L]) * kGridCB;
  const int nc = min(kGridCB, lv.C - c0);
  const uint32_t ucells = static_cast<uint32_t>(cells), uhw = static_cast<uint32_t>(HW);
  const uint32_t total = static_cast<uint32_t>(nc) * ucells;
  const float *__restrict__ ev = lv.events;
  float *__restrict__ grid = lv.grid;
  for (uint32_t t0 = tid; t0 < total; t0 += kGridThreads * kGridPer) {
    float v[kGridPer];
    int64_t o[kGridPer];
#pragma unroll
    for (int u = 0; u < kGridPer; ++u) {
      const uint32_t t = t0 + u * kGridThreads;
      o[u] = -1;
      v[u] = 0.f;
      if (t < total) {
        const uint32_t cl = t / ucells, cell = t - cl * ucells;
        const uint32_t b = cell / uhw, hw = cell - b * uhw;
        const int c = c0 + static_cast<int>(cl);
        const int32_t e = cell_ev[cell];
        o[u] = (static_cast<int64_t>(b) * lv.C + c) * HW + hw;
        if (e >= 0) v[u] = ev[static_cast<int64_t>(e) * lv.C + c];
      }
    }
#pragma unroll
    for (int u = 0; u < kGridPer; ++u)
      if (o[u] >= 0) grid[o[u]] = v[u];
  }
  const int any_bad = __syncthreads_or(bad ? 1 : 0);
  if (status && any_bad && tid == 0) *status = 1;
}

}  // namespace
}  // namespace ssla

using namespace ssla;

// ======================================================================== C-ABI
extern "C" int ssla_rf_lut_shape(int H, int W, int kh, int kw, int sh, int sw, int64_t *n_rf) {
  clear_error();
  SSLA_CHECK_ARG(H > 0 && W > 0 && kh > 0 && kw > 0 && sh > 0 && sw > 0 && n_rf, "rf_lut_shape: bad sizes");
  const int ph = ((H + sh - 1) / sh - 1) * sh + kh - H, pw = ((W + sw - 1) / sw - 1) * sw + kw - W;
  const int Ho = (H + ph - kh) / sh + 1, Wo = (W + pw - kw) / sw + 1;
  SSLA_CHECK_ARG(Ho > 0 && Wo > 0, "rf_lut_shape: empty output grid");
  *n_rf = static_cast<int64_t>(Ho) * Wo;
  return SSLA_OK;
}

extern "C" int ssla_rf_lut(int H, int W, int kh, int kw, int sh, int sw, int64_t *lut, int64_t *outcoord,
                           void *stream) {
  clear_error();
  int64_t n_rf = 0;
  const int st0 = ssla_rf_lut_shape(H, W, kh, kw, sh, sw, &n_rf);
  if (st0 != SSLA_OK) return st0;
  SSLA_CHECK_ARG(lut != nullptr, "rf_lut: lut is NULL");
  const int ph = ((H + sh - 1) / sh - 1) * sh + kh - H, pw = ((W + sw - 1) / sw - 1) * sw + kw - W;
  // floor(p / 2) for the top/left padding (p may be negative: a crop)
  const int top = ph >= 0 ? ph / 2 : -((-ph + 1) / 2), left = pw >= 0 ? pw / 2 : -((-pw + 1) / 2);
  const int Ho = (H + ph - kh) / sh + 1, Wo = (W + pw - kw) / sw + 1;
  hipLaunchKernelGGL(lut_kernel, dim3(grid_for(n_rf * kh * kw)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     H, W, kh, kw, sh, sw, top, left, Ho, Wo, lut, outcoord);
  return launch_status("rf_lut");
}

// ---- group_events ------------------------------------------------------------
namespace {
struct GeWs {
  int64_t *counts, *off, *head, *gpos, *start, *kept, *kpre, *row_of;
  uint64_t *key, *skey;
  int32_t *val, *order, *bad;
  uint64_t *lb;   // two look-back scan states of lb_state_words(cap) words
  int64_t lb_words;
  // the pixel sort (caps up to kRsMaxCap): one histogram (int32, up to
  // 2^12 digits per tile), its prefix, the first pass's output and a
  // look-back state per pass
  int32_t *rs_hist, *rs_tval;
  int64_t *rs_off;
  uint64_t *rs_tkey, *rs_lb;
  int64_t rs_tiles, rs_counters, rs_lb_words;
  void *tmp;
  size_t tmp_bytes, total;
};
constexpr int64_t kRsMaxCap = int64_t{1} << 21;
constexpr int kRsMaxDigit = 12;   // two passes cover keys up to 24 bits
GeWs ge_layout(void *ws, int B, int64_t cap) {
  Carve c{static_cast<char *>(ws)};
  GeWs L;
  L.counts = c.take<int64_t>(8);
  L.bad = c.take<int32_t>(8);
  L.off = c.take<int64_t>(B + 1);
  L.head = c.take<int64_t>(cap);
  L.gpos = c.take<int64_t>(cap);
  L.start = c.take<int64_t>(cap + 1);
  L.kept = c.take<int64_t>(cap);
  L.kpre = c.take<int64_t>(cap);
  L.row_of = c.take<int64_t>(cap);
  L.key = c.take<uint64_t>(cap);
  L.skey = c.take<uint64_t>(cap);
  L.val = c.take<int32_t>(cap);
  L.order = c.take<int32_t>(cap);
  L.lb_words = lb_state_words(cap);
  const bool rs = cap <= kRsMaxCap;
  L.rs_tiles = (cap + kRsTile - 1) / kRsTile;
  L.rs_counters = rs ? (int64_t{1} << kRsMaxDigit) * L.rs_tiles : 0;
  L.rs_lb_words = rs ? lb_state_words(L.rs_counters) : 0;
  // the scan states of the grouping (2) and of the pixel sort (2), contiguous
  L.lb = c.take<uint64_t>(2 * (L.lb_words + L.rs_lb_words));
  L.rs_lb = L.lb ? L.lb + 2 * L.lb_words : nullptr;
  L.rs_hist = c.take<int32_t>(L.rs_counters);
  L.rs_off = c.take<int64_t>(L.rs_counters);
  L.rs_tkey = c.take<uint64_t>(rs ? cap : 0);
  L.rs_tval = c.take<int32_t>(rs ? cap : 0);
  L.tmp_bytes = std::max(rs ? 0 : sort_temp_bytes(cap), scan_temp_bytes(std::max<int64_t>(cap, B + 1)));
  L.tmp = c.take<char>(L.tmp_bytes);
  L.total = c.off;
  return L;
}
}  // namespace

extern "C" size_t ssla_group_events_workspace_size(int B, int64_t N) {
  if (B <= 0 || N < 0) return 0;
  return ge_layout(nullptr, B, static_cast<int64_t>(B) * N).total;
}

namespace {
// group_events with the kept window (latest max_per_px, then the first
// keep_first), features from column fc and, with delays, the per-pixel
// delays of MosModel.preprocess_inputs in column fc.
int group_events_impl(const char *what, const float *events, const int64_t *lengths, int B, int64_t N, int C, int H,
                      int W, int max_per_px, int64_t keep_first, int fc, bool delays, float *out_events,
                      int64_t *out_time, int64_t *gr_batch, int64_t *gr_h, int64_t *gr_w, int64_t *gr_len,
                      void *workspace, size_t workspace_bytes, void *stream) {
  SSLA_CHECK_ARG(B > 0 && N >= 0 && C >= 4 && H > 0 && W > 0 && max_per_px > 0, "%s: bad sizes", what);
  SSLA_CHECK_ARG(static_cast<int64_t>(B) * H * W < (1LL << 24),
                 "%s: B*H*W must stay below 2^24 (pixel ids are formed in fp32)", what);
  const int64_t cap = static_cast<int64_t>(B) * N;
  SSLA_CHECK_ARG(cap < 0x7fffffff, "%s: B*N must stay below 2^31", what);
  const GeWs L = ge_layout(workspace, B, cap);
  if (!workspace || workspace_bytes < L.total) {
    set_error("%s: workspace of %zu bytes needed, %zu given", what, L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(events && lengths && out_events && out_time && gr_batch && gr_h && gr_w && gr_len,
                 "%s: null pointer", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t *Ep = L.off + B;
  if (cap == 0) {
    hipLaunchKernelGGL(clear_and_fill, dim3(1), dim3(kThreads), 0, st, L.counts, L.bad, nullptr, (int64_t)0,
                       (int64_t)0, nullptr, (int64_t)0, 0, nullptr, (int64_t)0);
    return launch_status(what);
  }
  // sample offsets: exclusive scan of the lengths clamped to [0, N], their
  // sum E in counts[2]
  // the pixel sort: two stable counting passes over digits of d1 and d2 bits
  // (keys up to n_pix, below 2^24) while the capacity is at most kRsMaxCap,
  // else rocPRIM's radix sort
  const int64_t n_pix = static_cast<int64_t>(B) * H * W;
  const bool rs = cap <= kRsMaxCap;
  const int bits = bits_for(static_cast<uint64_t>(n_pix));
  const int d1 = (bits + 1) / 2, d2 = bits - d1;
  const int64_t n_hist1 = rs ? (int64_t{1} << d1) * L.rs_tiles : 0;
  const int64_t n_lb = 2 * (L.lb_words + L.rs_lb_words);
  hipLaunchKernelGGL(clear_and_fill, dim3(grid_for(std::max(std::max<int64_t>(8, B + 1), std::max(n_lb, n_hist1)))),
                     dim3(kThreads), 0, st, L.counts, L.bad, L.kept, (int64_t)(B + 1), (int64_t)0, L.rs_hist, n_hist1,
                     0, nullptr, (int64_t)0, L.lb, n_lb);
  int s = SSLA_OK;
  if (B + 1 <= kSmallScan) {
    excl_scan_launch(TruncIn{lengths, B, N}, L.off, B + 1, nullptr, L.counts + 2, st);
  } else {
    hipLaunchKernelGGL(trunc_len, dim3(grid_for(B)), dim3(kThreads), 0, st, lengths, (int64_t)B, N, L.kept);
    s = excl_scan(L.tmp, L.tmp_bytes, L.kept, L.off, B + 1, st, nullptr, L.counts + 2);
    if (s) return s;
  }
  // keys of the valid events (pixel ids < B*H*W); padding slots take the key
  // B*H*W and sort last, so only the bits of B*H*W need sorting
  hipLaunchKernelGGL(ge_keys, dim3(grid_for(cap)), dim3(kThreads), 0, st, events, lengths, L.off, B, N, C, H, W,
                     L.key, L.val, L.row_of, L.bad, rs ? L.rs_hist : nullptr, d1, L.rs_tiles);
  if (rs) {
    excl_scan_launch(HistIn{L.rs_hist}, L.rs_off, n_hist1, L.rs_lb, nullptr, st);
    if (d2 > 0) {
      rs_pass<true>(L.key, L.val, cap, L.rs_tiles, 0, d1, L.rs_off, L.rs_tkey, L.rs_tval, d1, d2, L.rs_hist, st);
      excl_scan_launch(HistIn{L.rs_hist}, L.rs_off, (int64_t{1} << d2) * L.rs_tiles, L.rs_lb + L.rs_lb_words, nullptr,
                       st);
      rs_pass<false>(L.rs_tkey, L.rs_tval, cap, L.rs_tiles, d1, d2, L.rs_off, L.skey, L.order, 0, 0, nullptr, st);
    } else {
      rs_pass<false>(L.key, L.val, cap, L.rs_tiles, 0, d1, L.rs_off, L.skey, L.order, 0, 0, nullptr, st);
    }
  } else {
    s = sort_pairs(L.tmp, L.tmp_bytes, L.key, L.skey, L.val, L.order, cap, bits, st);
    if (s) return s;
  }
  // group heads (computed inside the scan) and their positions
  excl_scan_launch(SortedHeadsIn{L.skey, Ep, L.head}, L.gpos, cap, L.lb, nullptr, st);
  hipLaunchKernelGGL(ge_starts, dim3(grid_for(cap)), dim3(kThreads), 0, st, L.head, L.gpos, cap, Ep, L.start,
                     L.counts);
  hipLaunchKernelGGL(ge_groups, dim3(grid_for(cap)), dim3(kThreads), 0, st, L.counts, L.start, cap, L.order,
                     L.row_of, events, N, C, max_per_px, keep_first, L.kept, gr_batch, gr_h, gr_w, gr_len);
  // kept-event offsets, their sum in counts[1]
  s = excl_scan(L.tmp, L.tmp_bytes, L.kept, L.kpre, cap, st, L.lb + L.lb_words, L.counts + 1);
  if (s) return s;
  if (delays)
    hipLaunchKernelGGL(ge_emit<true>, dim3(grid_for(cap)), dim3(kThreads), 0, st, L.head, L.gpos, L.start, L.kept,
                       L.kpre, L.order, L.row_of, events, cap, Ep, C, max_per_px, fc, out_events, out_time);
  else
    hipLaunchKernelGGL(ge_emit<false>, dim3(grid_for(cap)), dim3(kThreads), 0, st, L.head, L.gpos, L.start, L.kept,
                       L.kpre, L.order, L.row_of, events, cap, Ep, C, max_per_px, fc, out_events, out_time);
  return launch_status(what);
}
}  // namespace

extern "C" int ssla_group_events(const float *events, const int64_t *lengths, int B, int64_t N, int C, int H, int W,
                                 int max_per_px, float *out_events, int64_t *out_time, int64_t *gr_batch,
                                 int64_t *gr_h, int64_t *gr_w, int64_t *gr_len, void *workspace,
                                 size_t workspace_bytes, void *stream) {
  clear_error();
  return group_events_impl("group_events", events, lengths, B, N, C, H, W, max_per_px, INT64_MAX, 3, false,
                           out_events, out_time, gr_batch, gr_h, gr_w, gr_len, workspace, workspace_bytes, stream);
}

// MosModel.preprocess_inputs in one call: out_events [cap, C - 2] holds
// (delay, features after t) per kept event.
extern "C" int ssla_preprocess_events(const float *events, const int64_t *lengths, int B, int64_t N, int C, int H,
                                      int W, int max_per_px, int64_t hot_pixel_thres, float *out_events,
                                      int64_t *out_time, int64_t *gr_batch, int64_t *gr_h, int64_t *gr_w,
                                      int64_t *gr_len, void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  return group_events_impl("preprocess_events", events, lengths, B, N, C, H, W, max_per_px,
                           hot_pixel_thres > 0 ? hot_pixel_thres : INT64_MAX, 2, true, out_events, out_time, gr_batch,
                           gr_h, gr_w, gr_len, workspace, workspace_bytes, stream);
}

// counts of the last data-dependent call that used `workspace` (the first
// n_counts int64 of the workspace) and its status flag; synchronises stream.
extern "C" int ssla_events_counts(const void *workspace, int64_t *counts_out, int n_counts, int *bad_out,
                                  void *stream) {
  clear_error();
  SSLA_CHECK_ARG(workspace && counts_out && n_counts > 0 && n_counts <= 8, "events_counts: bad arguments");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // counts at byte 0, the bad-input flag at byte 256: one read covers both
  unsigned char raw[256 + sizeof(int32_t)];
  const hipError_t e = read_to_host(raw, workspace, sizeof(raw), st);
  if (e != hipSuccess) {
    set_error("events_counts: %s", hipGetErrorString(e));
    return SSLA_ERR_LAUNCH;
  }
  int64_t buf[8];
  int32_t badv[1];
  memcpy(buf, raw, sizeof(buf));
  memcpy(badv, raw + 256, sizeof(badv));
  for (int i = 0; i < n_counts; ++i) counts_out[i] = buf[i];
  if (bad_out) *bad_out = badv[0];
  return SSLA_OK;
}

// The counts head of a workspace (the 260 bytes ssla_events_counts reads)
// copied into host memory in stream order, without waiting: host_head must
// be pinned (page-locked) memory; the copy has landed once the stream has
// passed this point (an event recorded after the call).
extern "C" int ssla_events_counts_async(const void *workspace, void *host_head, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(workspace && host_head, "events_counts_async: null pointer");
  const hipError_t e = hipMemcpyAsync(host_head, workspace, 256 + sizeof(int32_t), hipMemcpyDeviceToHost,
                                      static_cast<hipStream_t>(stream));
  if (e != hipSuccess) {
    set_error("events_counts_async: %s", hipGetErrorString(e));
    return SSLA_ERR_LAUNCH;
  }
  return SSLA_OK;
}

// ---- receptive-field / patch scatter without a sort --------------------------------
// When every pixel run is non-decreasing in time (clamped at 0, the sort
// key), the stable (field, time) order is fixed by counting: event i of the
// run at kernel position a of field f lands on row
//   ev_pre[f] + i + sum_{a' < a} #(run a' <= t) + sum_{a' > a} #(run a' < t),
// exactly where the stable sort of rf_enumerate's keys puts it (ties keep
// the enumeration order: position, then run order).
namespace {
// ev2g[e] = g for the events e of group g's run (when store; one thread
// per event, its group found by binary search over the run starts gstart,
// the exclusive prefix of the run lengths), and n_bad > 0 if a run is not
// non-decreasing in time (clamped at 0: one count per decreasing pair) or
// leaves [0, E_in) (one count per such run).  Without store (ev2g too small)
// one thread adds 1, which sends the caller to the sort fill.
__global__ void rf_groups_scan(const int64_t *__restrict__ gstart, const int64_t *__restrict__ glen, int64_t G,
                               const int64_t *__restrict__ time, int64_t E_in, int32_t *__restrict__ ev2g, int store,
                               unsigned long long *__restrict__ n_bad) {
  if (!store) {
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(n_bad, 1ull);
    return;
  }
  GRID_STRIDE(e, E_in) {
    const int64_t g = last_le(gstart, G, e);
    const int64_t s = gstart[g];
    if (e >= s && e < s + glen[g]) {
      ev2g[e] = static_cast<int32_t>(g);
      if (e > s && max(time[e], (int64_t)0) < max(time[e - 1], (int64_t)0)) atomicAdd(n_bad, 1ull);
    }
  }
  GRID_STRIDE(g, G) {
    const int64_t s = gstart[g], n = glen[g];
    if (n > 0 && (s < 0 || s + n > E_in)) atomicAdd(n_bad, 1ull);
  }
}

// inv[p * A + a] = rf with lut[rf * A + a] == p (each (pixel, position)
// pair belongs to at most one field)
__global__ void rf_inv_lut(const int64_t *__restrict__ lut, int64_t n_rf, int A, int64_t HW,
                           int32_t *__restrict__ inv) {
  GRID_STRIDE(t, n_rf * A) {
    const int64_t p = lut[t];
    if (p >= 0 && p < HW) inv[p * A + t % A] = static_cast<int32_t>(t / A);
  }
}

// One thread per (event, kernel position).  o_time, o_pos, dst_map and
// o_fidx (the row's active-field index, act_pre of its field) are optional.
template <bool ONE>
__global__ void rf_merge(const int32_t *__restrict__ ev2g, const int64_t *__restrict__ gb,
                         const int64_t *__restrict__ gh, const int64_t *__restrict__ gw,
                         const int64_t *__restrict__ gstart, const int64_t *__restrict__ glen,
                         const int32_t *__restrict__ pixmap, const int32_t *__restrict__ inv,
                         const int64_t *__restrict__ lut, int64_t n_rf, int A, int B, int H, int W,
                         const int64_t *__restrict__ ev_pre, const int64_t *__restrict__ time, int64_t E_in,
                         int64_t E_out, int64_t *__restrict__ o_src, int64_t *__restrict__ o_time,
                         int64_t *__restrict__ o_pos, int32_t *__restrict__ dst_map,
                         const int64_t *__restrict__ act_pre, int32_t *__restrict__ o_fidx) {
  const int64_t HW = static_cast<int64_t>(H) * W;
  // ONE: one thread per event, its only (field, position) from inv[p]
  // (every pixel in at most one field); else one per (event, position)
  GRID_STRIDE(t, ONE ? E_in : E_in * A) {
    // E_in * A < 2^31 (checked by the callers): 32-bit division, not the
    // 64-bit emulation
    const uint32_t t32 = static_cast<uint32_t>(t);
    const int64_t e = ONE ? t : static_cast<int64_t>(t32 / static_cast<uint32_t>(A));
    int a = ONE ? 0 : static_cast<int>(t32 - static_cast<uint32_t>(e) * static_cast<uint32_t>(A));
    const int32_t g = ev2g[e];
    if (g < 0) continue;
    const int64_t b = gb[g], p = gh[g] * W + gw[g];
    // (inputs the plan reports as bad are only kept in range here: the
    // counting fill may run before the plan's counts are read)
    if (b < 0 || b >= B || p < 0 || p >= HW) continue;
    int32_t rf;
    if constexpr (ONE) {
      const int32_t pf = inv[p];
      if (pf < 0) continue;
      rf = static_cast<int32_t>(static_cast<uint32_t>(pf) / static_cast<uint32_t>(A));
      a = pf - rf * A;
    } else {
      rf = inv[p * A + a];
      if (rf < 0) continue;
    }
    const int64_t tt = max(time[e], (int64_t)0);
    int64_t rank = e - gstart[g];
    // the other positions kMB at a time: their table entries, groups and
    // runs are loaded side by side, then their binary searches advance in
    // lockstep, so the chain of dependent loads is about as long as one
    // position's instead of the sum over all of them
    constexpr int kMB = 8;
    for (int a0 = 0; a0 < A; a0 += kMB) {
      int64_t p2[kMB];
#pragma unroll
      for (int u = 0; u < kMB; ++u) {
        const int a2 = a0 + u;
        p2[u] = (a2 < A && a2 != a) ? lut[static_cast<int64_t>(rf) * A + a2] : -1;
      }
      int32_t g2[kMB];
#pragma unroll
      for (int u = 0; u < kMB; ++u) g2[u] = p2[u] >= 0 ? pixmap[b * HW + p2[u]] : -1;
      int64_t s2[kMB];
      int32_t lo[kMB], hi[kMB];
#pragma unroll
      for (int u = 0; u < kMB; ++u) {
        s2[u] = g2[u] >= 0 ? min(max(gstart[g2[u]], (int64_t)0), E_in) : 0;
        lo[u] = 0;
        hi[u] = g2[u] >= 0 ? static_cast<int32_t>(min(max(glen[g2[u]], (int64_t)0), E_in - s2[u])) : 0;
      }
      bool more = true;
      while (more) {
        more = false;
#pragma unroll
        for (int u = 0; u < kMB; ++u) {
          if (lo[u] < hi[u]) {   // elements < tt (<= tt for earlier positions), times clamped at 0
            const int32_t mid = (lo[u] + hi[u]) >> 1;
            const int64_t v = max(time[s2[u] + mid], (int64_t)0);
            const bool le = a0 + u < a ? v <= tt : v < tt;
            lo[u] = le ? mid + 1 : lo[u];
            hi[u] = le ? hi[u] : mid;
            more = true;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kMB; ++u) rank += lo[u];
    }
    const int64_t row = ev_pre[b * n_rf + rf] + rank;
    if (row < 0 || row >= E_out) continue;   // inconsistent inputs: drop, never write out of range
    o_src[row] = e;
    if (o_time) o_time[row] = time[e];
    if (o_pos) o_pos[row] = a;
    if (dst_map) dst_map[e * A + a] = static_cast<int32_t>(row);
    if (o_fidx) o_fidx[row] = static_cast<int32_t>(act_pre[b * n_rf + rf]);
  }
}
}  // namespace

// ---- receptive-field / patch scatter ---------------------------------------------
namespace {
struct RfWs {
  int64_t *counts, *gstart, *nev, *act, *act_pre, *ev_pre, *f_index, *f_len, *pre_src, *pre_pos, *pk, *pk_pre;
  int32_t *bad, *pixmap, *val, *perm;
  uint64_t *key, *skey;
  unsigned long long *tmax;
  // look-back scan states (zeroed by the plan's set-up kernel): the group
  // starts' scan (lb_state_words(G)) and the segment heads' scan of the
  // pooling plan (lb_state_words(E_cap)), contiguous
  uint64_t *lb_g, *lb_e, *lb_c;
  int64_t lb_words;
  void *tmp;
  size_t tmp_bytes, total;
};
RfWs rf_layout(void *ws, int64_t G, int64_t n_pix, int64_t n_f, int64_t E_cap) {
  Carve c{static_cast<char *>(ws)};
  RfWs L;
  L.counts = c.take<int64_t>(8);
  L.bad = c.take<int32_t>(8);
  L.tmax = c.take<unsigned long long>(1);
  L.gstart = c.take<int64_t>(G + 1);
  L.pixmap = c.take<int32_t>(n_pix);
  L.nev = c.take<int64_t>(n_f);
  L.act = c.take<int64_t>(n_f);
  L.act_pre = c.take<int64_t>(n_f);
  L.ev_pre = c.take<int64_t>(n_f);
  L.f_index = c.take<int64_t>(n_f);
  L.f_len = c.take<int64_t>(n_f);
  L.pk = c.take<int64_t>(n_f);
  L.pk_pre = c.take<int64_t>(n_f);
  L.pre_src = c.take<int64_t>(E_cap);
  L.pre_pos = c.take<int64_t>(E_cap);
  L.key = c.take<uint64_t>(E_cap);
  L.skey = c.take<uint64_t>(E_cap);
  L.val = c.take<int32_t>(E_cap);
  L.perm = c.take<int32_t>(E_cap);
  // (and the fused field count's: one flag per 256 (field, position) lanes)
  L.lb_words = lb_state_words(G) + lb_state_words(E_cap) + 2 + (n_f * 64 + 255) / 256;
  L.lb_g = c.take<uint64_t>(L.lb_words);
  L.lb_e = L.lb_g ? L.lb_g + lb_state_words(G) : nullptr;
  L.lb_c = L.lb_e ? L.lb_e + lb_state_words(E_cap) : nullptr;
  L.tmp_bytes = std::max(sort_temp_bytes(E_cap), scan_temp_bytes(std::max(n_f, G + 1)));
  L.tmp = c.take<char>(L.tmp_bytes);
  L.total = c.off;
  return L;
}
}  // namespace

// E_cap bounds the number of field events (sum over active fields of their
// pixels' runs; at most A * E_in).
extern "C" size_t ssla_rf_scatter_workspace_size(int64_t G, int B, int H, int W, int64_t n_rf, int64_t E_cap) {
  if (G < 0 || B <= 0 || H <= 0 || W <= 0 || n_rf <= 0 || E_cap < 0) return 0;
  return rf_layout(nullptr, G, static_cast<int64_t>(B) * H * W, static_cast<int64_t>(B) * n_rf, E_cap).total;
}

// Plan: which (b, rf) fields are active and how many events each holds.
// counts[0] = active fields, counts[1] = field events, counts[2] = max time,
// counts[3] = pixel runs that are not non-decreasing in time (0: the
// sort-free fill applies).
namespace {
// The plan; inv (H * W * A int32, or NULL) also receives the inverse table of
// the counting fill in the same launches, and with_tmax = false leaves
// counts[2] (the largest time, which only the sort fill needs) at 0.
int rf_plan_impl(const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w, const int64_t *gr_len, int64_t G,
                 const int64_t *time, int64_t E_in, int B, int H, int W, const int64_t *lut, int64_t n_rf, int A,
                 int64_t E_cap, int32_t *inv, bool one_field, bool with_tmax, void *workspace,
                 size_t workspace_bytes, hipStream_t st) {
  SSLA_CHECK_ARG(G >= 0 && E_in >= 0 && B > 0 && H > 0 && W > 0 && n_rf > 0 && A > 0 && E_cap >= 0,
                 "rf_scatter_plan: bad sizes");
  SSLA_CHECK_ARG(E_cap < 0x7fffffff, "rf_scatter_plan: E_cap must stay below 2^31");
  const int64_t n_pix = static_cast<int64_t>(B) * H * W, n_f = static_cast<int64_t>(B) * n_rf;
  const RfWs L = rf_layout(workspace, G, n_pix, n_f, E_cap);
  if (!workspace || workspace_bytes < L.total) {
    set_error("rf_scatter_plan: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(lut && (G == 0 || (gr_batch && gr_h && gr_w && gr_len)) && (E_in == 0 || time),
                 "rf_scatter_plan: null pointer");
  const int64_t n_inv = inv ? static_cast<int64_t>(H) * W * (one_field ? 1 : A) : 0;
  // event -> group table (the sort-free fill's input; kept in the value
  // buffer of the sort path, which needs E_in <= E_cap): -1 until
  // rf_groups_scan fills it
  const int store = E_in <= E_cap;
  const int64_t n_ev2g = store ? E_in : 0;
  hipLaunchKernelGGL(clear_and_fill,
                     dim3(grid_for(std::max(std::max(std::max<int64_t>(8, n_pix), std::max(n_inv, n_ev2g)),
                                            L.lb_words))),
                     dim3(kThreads), 0, st, L.counts, L.bad, reinterpret_cast<int64_t *>(L.tmax), (int64_t)1,
                     (int64_t)0, L.pixmap, n_pix, -1, inv, n_inv, L.lb_g, L.lb_words, L.val, n_ev2g);
  if (G > 0 || inv)
    hipLaunchKernelGGL(rf_pixmap, dim3(grid_for(std::max(G, inv ? n_rf * A : 0))), dim3(kThreads), 0, st, gr_batch,
                       gr_h, gr_w, G, H, W, n_pix, L.pixmap, L.bad, lut, n_rf, A, inv, one_field ? 1 : 0,
                       L.counts + 5);
  int s = excl_scan(L.tmp, L.tmp_bytes, gr_len, L.gstart, G, st, L.lb_g);
  if (s) return s;
  // one prefix sum of the packed (events, active) pairs while the active
  // count fits 21 bits
  const bool packed = n_f < (int64_t{1} << kPackBits);
  const bool lanes = 64 % A == 0 && n_f * A <= (int64_t{1} << 28);
  if (packed && lanes && n_f > 0) {   // count, prefix and compaction in one launch
    hipLaunchKernelGGL(rf_count_scan, dim3(static_cast<unsigned>((n_f * A + 255) / 256)), dim3(256), 0, st, lut, n_rf,
                       A, B, H, W, L.pixmap, gr_len, L.nev, L.act, L.act_pre, L.ev_pre, L.f_index, L.f_len, L.counts,
                       L.lb_c);
  } else if (lanes)
    hipLaunchKernelGGL(rf_count_lanes, dim3(static_cast<unsigned>((n_f * A + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, st, lut, n_rf, A, B, H, W, L.pixmap, gr_len, L.nev, L.act,
                       packed ? L.pk : nullptr);
  else
    hipLaunchKernelGGL(rf_count, dim3(grid_for(n_f)), dim3(kThreads), 0, st, lut, n_rf, A, B, H, W, L.pixmap, gr_len,
                       L.nev, L.act, packed ? L.pk : nullptr);
  if (packed && lanes && n_f > 0) {
    // done above
  } else if (packed) {
    s = excl_scan(L.tmp, L.tmp_bytes, L.pk, L.pk_pre, n_f, st);
    if (s) return s;
    hipLaunchKernelGGL(rf_unpack_fields, dim3(grid_for(n_f)), dim3(kThreads), 0, st, L.pk_pre, L.pk, n_f, L.act_pre,
                       L.ev_pre, L.counts, L.f_index, L.f_len);
  } else {
    s = excl_scan(L.tmp, L.tmp_bytes, L.act, L.act_pre, n_f, st);
    if (s) return s;
    s = excl_scan(L.tmp, L.tmp_bytes, L.nev, L.ev_pre, n_f, st);
    if (s) return s;
    hipLaunchKernelGGL(total_from_scan, dim3(1), dim3(64), 0, st, L.act_pre, L.act, n_f, L.counts + 0);
    hipLaunchKernelGGL(total_from_scan, dim3(1), dim3(64), 0, st, L.ev_pre, L.nev, n_f, L.counts + 1);
  }
  if (E_in > 0 && with_tmax)
    hipLaunchKernelGGL(max_i64, dim3(grid_for(std::min<int64_t>(E_in, 1 << 16))), dim3(kThreads), 0, st, time, E_in,
                       L.tmax);
  if (!packed)
    hipLaunchKernelGGL(rf_fields, dim3(grid_for(n_f)), dim3(kThreads), 0, st, L.act, L.act_pre, L.nev, n_f, L.f_index,
                       L.f_len);
  if (with_tmax) hipLaunchKernelGGL(store_u64_as_i64, dim3(1), dim3(64), 0, st, L.tmax, L.counts + 2);
  // the event -> group table and the count of unsorted runs
  if (G > 0 || !store)
    hipLaunchKernelGGL(rf_groups_scan, dim3(grid_for(std::max<int64_t>(std::max(G, E_in), 1))), dim3(kThreads), 0,
                       st, L.gstart, gr_len, G, time, E_in, L.val, store,
                       reinterpret_cast<unsigned long long *>(L.counts + 3));
  return launch_status("rf_scatter_plan");
}
}  // namespace

extern "C" int ssla_rf_scatter_plan(const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w,
                                    const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in, int B,
                                    int H, int W, const int64_t *lut, int64_t n_rf, int A, int64_t E_cap,
                                    void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  return rf_plan_impl(gr_batch, gr_h, gr_w, gr_len, G, time, E_in, B, H, W, lut, n_rf, A, E_cap, nullptr, false,
                      true, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

// Fill (after the plan; n_active / E_out / t_max are the plan's counts):
// field events in (field, time) order with their source pixel event, time
// and kernel position; per active field its flat (b, rf) index and length.
extern "C" int ssla_rf_scatter_fill(const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in, int B,
                                    int H, int W, const int64_t *lut, int64_t n_rf, int A, int64_t E_cap,
                                    int64_t n_active, int64_t E_out, int64_t t_max, int64_t *out_src,
                                    int64_t *out_time, int64_t *out_pos, int64_t *f_index, int64_t *f_len,
                                    void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  const int64_t n_pix = static_cast<int64_t>(B) * H * W, n_f = static_cast<int64_t>(B) * n_rf;
  const RfWs L = rf_layout(workspace, G, n_pix, n_f, E_cap);
  if (!workspace || workspace_bytes < L.total) {
    set_error("rf_scatter_fill: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(E_out >= 0 && E_out <= E_cap && n_active >= 0 && n_active <= n_f && t_max >= 0,
                 "rf_scatter_fill: counts outside the plan's capacity");
  SSLA_CHECK_ARG(out_src && out_pos && f_index && f_len, "rf_scatter_fill: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t t_stride = static_cast<uint64_t>(t_max) + 1;
  hipLaunchKernelGGL(rf_enumerate, dim3(grid_for(n_f * A)), dim3(kThreads), 0, st, lut, n_rf, A, B, H, W, L.pixmap,
                     gr_len, L.gstart, L.act, L.act_pre, L.ev_pre, time, E_in, t_stride, L.key, L.val, L.pre_src,
                     L.pre_pos);
  const int end_bit = bits_for(static_cast<uint64_t>(std::max<int64_t>(n_active, 1)) * t_stride);
  int s = sort_pairs(L.tmp, L.tmp_bytes, L.key, L.skey, L.val, L.perm, E_out, end_bit, st);
  if (s) return s;
  if (E_out > 0)
    hipLaunchKernelGGL(rf_emit, dim3(grid_for(E_out)), dim3(kThreads), 0, st, L.perm, E_out, L.pre_src, L.pre_pos,
                       time, out_src, out_time, out_pos, static_cast<const uint64_t *>(nullptr), t_stride,
                       static_cast<int32_t *>(nullptr));
  if (n_active > 0) {
    hipError_t e = hipMemcpyAsync(f_index, L.f_index, sizeof(int64_t) * n_active, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(f_len, L.f_len, sizeof(int64_t) * n_active, hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) {
      set_error("rf_scatter_fill: %s", hipGetErrorString(e));
      return SSLA_ERR_LAUNCH;
    }
  }
  return launch_status("rf_scatter_fill");
}


// Fill without a sort, for plans with counts[3] == 0 (every pixel run sorted
// by time): the same outputs as ssla_rf_scatter_fill, from the plan's event
// -> group table.  inv (H * W * A int32) is scratch the caller provides; dst_map
// (E_in * A int32, optional) receives the row of every (event, position)
// pair, -1 where the pair is in no field.
extern "C" int ssla_rf_scatter_fill_sorted(const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w,
                                           const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in,
                                           int B, int H, int W, const int64_t *lut, int64_t n_rf, int A,
                                           int64_t E_cap, int64_t n_active, int64_t E_out, int64_t *out_src,
                                           int64_t *out_time, int64_t *out_pos, int64_t *f_index, int64_t *f_len,
                                           int32_t *inv, int32_t *dst_map, void *workspace, size_t workspace_bytes,
                                           void *stream) {
  clear_error();
  const int64_t n_pix = static_cast<int64_t>(B) * H * W, n_f = static_cast<int64_t>(B) * n_rf;
  const RfWs L = rf_layout(workspace, G, n_pix, n_f, E_cap);
  if (!workspace || workspace_bytes < L.total) {
    set_error("rf_scatter_fill_sorted: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(E_out >= 0 && E_out <= E_cap && n_active >= 0 && n_active <= n_f && A > 0,
                 "rf_scatter_fill_sorted: counts outside the plan's capacity");
  SSLA_CHECK_ARG(out_src && out_pos && f_index && f_len && inv, "rf_scatter_fill_sorted: null pointer");
  SSLA_CHECK_ARG(E_in <= E_cap, "rf_scatter_fill_sorted: needs E_in <= E_cap (the plan's event table)");
  SSLA_CHECK_ARG(G == 0 || (gr_batch && gr_h && gr_w && gr_len), "rf_scatter_fill_sorted: null group arrays");
  SSLA_CHECK_ARG(E_out < 0x7fffffff && E_in * A < 0x7fffffff,
                 "rf_scatter_fill_sorted: E_out and E_in * A must stay below 2^31");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t HW = static_cast<int64_t>(H) * W;
  const int64_t n_dst = dst_map ? E_in * A : 0;
  const int64_t n_act = std::max<int64_t>(n_active, 0);
  hipLaunchKernelGGL(rf_sorted_setup, dim3(grid_for(std::max(std::max(HW * A, n_dst), n_act))), dim3(kThreads), 0, st,
                     inv, HW * A, dst_map, n_dst, f_index, L.f_index, f_len, L.f_len, n_act);
  hipLaunchKernelGGL(rf_inv_lut, dim3(grid_for(n_rf * A)), dim3(kThreads), 0, st, lut, n_rf, A, HW, inv);
  if (E_in > 0) {
    if (E_out > 0)
      hipLaunchKernelGGL(rf_merge<false>, dim3(grid_for(E_in * A)), dim3(kThreads), 0, st, L.val, gr_batch, gr_h, gr_w,
                         L.gstart, gr_len, L.pixmap, inv, lut, n_rf, A, B, H, W, L.ev_pre, time, E_in, E_out, out_src,
                         out_time, out_pos, dst_map, static_cast<const int64_t *>(nullptr),
                         static_cast<int32_t *>(nullptr));
  }
  return launch_status("rf_scatter_fill_sorted");
}

// ---- SparsePool in two calls --------------------------------------------------------
// SparsePool.forward (reference layers/sparse_pooling.py:14-48) with the
// receptive-field gather in front of it (utils/farsecnn_utils.py:177-265),
// for callers that need only the pooled sequences: the field rows are never
// stored as [rows, C] features -- the reduction reads the pixel events
// through each row's source index.
//   plan: the field plan, the (field, time)-ordered rows (source event,
//         time, active field), the segment heads (a field's first row, or
//         a time change inside a field) and their exclusive prefix sum.
//   emit: per segment the max or mean of its rows' features and its time;
//         per active field its segment count, batch, h and w.
namespace {
struct PoolWs {
  RfWs rf;
  int64_t *src, *tim, *head, *segx;
  int32_t *fidx, *inv;
  void *tmp;
  size_t tmp_bytes, total;
};
PoolWs pool_layout(void *ws, int64_t G, int B, int H, int W, int64_t n_rf, int A, int64_t E_cap) {
  PoolWs L;
  L.rf = rf_layout(ws, G, static_cast<int64_t>(B) * H * W, static_cast<int64_t>(B) * n_rf, E_cap);
  Carve c{static_cast<char *>(ws), L.rf.total};
  L.src = c.take<int64_t>(E_cap);
  L.tim = c.take<int64_t>(E_cap);
  L.head = c.take<int64_t>(E_cap);
  L.segx = c.take<int64_t>(E_cap);
  L.fidx = c.take<int32_t>(E_cap);
  L.inv = c.take<int32_t>(static_cast<int64_t>(H) * W * A);
  L.tmp_bytes = scan_temp_bytes(E_cap);
  L.tmp = c.take<char>(L.tmp_bytes);
  L.total = c.off;
  return L;
}

// head[r] = 1 where row r starts a pooling segment: the first row, a new
// field, or a time different from the row before (reference
// sparse_pooling.py:26-31: unique_consecutive of time + field * max_v).
// Rows at or past the row count *n_rows (read on the device) get 0, so the
// prefix sum may run over the capacity cap.
__global__ void pool_row_heads(const int32_t *__restrict__ fidx, const int64_t *__restrict__ tim,
                               const int64_t *__restrict__ n_rows, int64_t cap, int64_t *__restrict__ head) {
  const int64_t n = min(*n_rows, cap);
  GRID_STRIDE(r, cap) head[r] = (r < n && (r == 0 || fidx[r] != fidx[r - 1] || tim[r] != tim[r - 1])) ? 1 : 0;
}

// One thread per (row, channel); the threads of a segment's first row walk
// the segment.  MEAN: the fp64 sum in row order over the count, rounded
// once.  Max: the first row among equal maxima; NaN never wins; a segment
// whose values are all NaN gives 0 (scatter_max's rule for a row that no
// event wins).  Then per active field its segment count and coordinates.
// LIN: ev holds two inputs per event and a row's value is its bf16 linear
// map by w_lin (bf16 [C, 2]): both inputs and the result rounded to bf16
// (nearest-even), the two products exact in fp32 and their sum rounded
// once -- what a bf16 GEMM with fp32 accumulation returns for K = 2.
template <bool MEAN, int VW, bool LIN = false>
__global__ void pool_emit_rows(const float *__restrict__ ev, int64_t E_in, int C, const int64_t *__restrict__ src,
                               const int64_t *__restrict__ tim, const int64_t *__restrict__ head,
                               const int64_t *__restrict__ segx, int64_t E_out, int64_t n_seg,
                               const int64_t *__restrict__ f_index, const int64_t *__restrict__ f_len,
                               const int64_t *__restrict__ ev_pre, int64_t n_act, int64_t n_rf,
                               const int64_t *__restrict__ outcoord, float *__restrict__ o_ev,
                               int64_t *__restrict__ o_time, int64_t *__restrict__ o_len, int64_t *__restrict__ o_b,
                               int64_t *__restrict__ o_h, int64_t *__restrict__ o_w,
                               const uint16_t *__restrict__ w_lin = nullptr) {
  // VW consecutive channels per thread (C / VW threads per row; E_out * C
  // < 2^31, checked by the caller).  A null o_ev skips the values (the
  // structure alone: times, per-field counts and coordinates); a null o_len
  // skips the per-field outputs (the values, with the times if o_time).
  const uint32_t CV = static_cast<uint32_t>(C / VW);
  if (!o_ev) {
    if (o_time) {
      GRID_STRIDE(r, E_out) {
        const int64_t s = segx[r];
        if (head[r] && s >= 0 && s < n_seg) o_time[s] = tim[r];
      }
    }
  } else GRID_STRIDE(t, E_out * CV) {
    const uint32_t t32 = static_cast<uint32_t>(t);
    const int64_t r = static_cast<int64_t>(t32 / CV);
    const int c = static_cast<int>(t32 - static_cast<uint32_t>(r) * CV) * VW;
    if (!head[r]) continue;
    const int64_t s = segx[r];
    if (s < 0 || s >= n_seg) continue;
    double sum[VW];
    float best[VW];
    bool found[VW];
    float wl[VW][2];
#pragma unroll
    for (int v = 0; v < VW; ++v) {
      sum[v] = 0.0;
      best[v] = -INFINITY;
      found[v] = false;
      if constexpr (LIN) {
        wl[v][0] = bf16_bits_to_f32(w_lin[(c + v) * 2]);
        wl[v][1] = bf16_bits_to_f32(w_lin[(c + v) * 2 + 1]);
      }
    }
    int64_t r2 = r;
    do {
      const int64_t e = src[r2];
      float x[VW];
      if (e >= 0 && e < E_in) {
        if constexpr (LIN) {
          const float2 in = *reinterpret_cast<const float2 *>(ev + e * 2);
          const float a0 = bf16_bits_to_f32(f32_to_bf16_bits(in.x)), a1 = bf16_bits_to_f32(f32_to_bf16_bits(in.y));
#pragma unroll
          for (int v = 0; v < VW; ++v) x[v] = bf16_bits_to_f32(f32_to_bf16_bits(a0 * wl[v][0] + a1 * wl[v][1]));
        } else if constexpr (VW == 4) {
          const float4 q = *reinterpret_cast<const float4 *>(ev + e * C + c);
          x[0] = q.x, x[1] = q.y, x[2] = q.z, x[3] = q.w;
        } else {
#pragma unroll
          for (int v = 0; v < VW; ++v) x[v] = ev[e * C + c + v];
        }
      } else {
#pragma unroll
        for (int v = 0; v < VW; ++v) x[v] = 0.f;
      }
#pragma unroll
      for (int v = 0; v < VW; ++v) {
        if constexpr (MEAN) {
          sum[v] += static_cast<double>(x[v]);
        } else {
          const bool take = x[v] > best[v] || (!found[v] && x[v] == best[v]);
          best[v] = take ? x[v] : best[v];
          found[v] = found[v] || take;
        }
      }
      ++r2;
    } while (r2 < E_out && !head[r2]);
#pragma unroll
    for (int v = 0; v < VW; ++v) {
      if constexpr (MEAN) o_ev[s * C + c + v] = static_cast<float>(sum[v] / static_cast<double>(r2 - r));
      else o_ev[s * C + c + v] = found[v] ? best[v] : 0.f;
    }
    if (c == 0 && o_time) o_time[s] = tim[r];
  }
  if (o_len) GRID_STRIDE(j, n_act) {
    const int64_t f = f_index[j], len = f_len[j];
    const int64_t st = ev_pre[f];
    int64_t segs = 0;
    if (len > 0 && st >= 0 && st + len <= E_out) segs = segx[st + len - 1] + head[st + len - 1] - segx[st];
    const int64_t rf = f % n_rf;
    o_len[j] = segs;
    o_b[j] = f / n_rf;
    o_h[j] = outcoord[rf * 2 + 1];
    o_w[j] = outcoord[rf * 2];
  }
}

// Segment heads of the filled field rows, their exclusive prefix and the
// segment count (workspace head, slot 4).  first: the plan's first pass,
// whose set-up kernel zeroed the look-back scan state (a second pass, after
// the sort fill, takes rocPRIM's scan).
int pool_segments_pass(const PoolWs &L, int64_t E_cap, hipStream_t st, bool first) {
  if (first && E_cap > 0) {   // the head flags computed inside the scan's launch
    excl_scan_launch(RowHeadsIn{L.fidx, L.tim, L.rf.counts + 1, E_cap, L.head}, L.segx, E_cap, L.rf.lb_e,
                     L.rf.counts + 4, st);
    return SSLA_OK;
  }
  hipLaunchKernelGGL(pool_row_heads, dim3(grid_for(E_cap)), dim3(kThreads), 0, st, L.fidx, L.tim, L.rf.counts + 1,
                     E_cap, L.head);
  return excl_scan(L.tmp, L.tmp_bytes, L.head, L.segx, E_cap, st, nullptr, L.rf.counts + 4);
}
}  // namespace

// E_cap bounds the field rows: E_in times the fields a pixel can belong to
// (ceil(kh / sh) * ceil(kw / sw) for a k x k, stride s field grid).
extern "C" size_t ssla_sparse_pool_workspace_size(int64_t G, int64_t E_in, int B, int H, int W, int64_t n_rf, int A,
                                                  int64_t E_cap) {
  if (G < 0 || E_in < 0 || B <= 0 || H <= 0 || W <= 0 || n_rf <= 0 || A <= 0 || E_cap < E_in) return 0;
  return pool_layout(nullptr, G, B, H, W, n_rf, A, E_cap).total;
}

// The plan's kernels up to the segment count, with no read back: the
// counts land in the workspace's head (ssla_events_counts layout).  The
// rows are filled by counting, on the premise that every pixel run is
// sorted by time (as group_events and pooled outputs leave them), and the
// segment heads and their prefix sum run over the capacity E_cap, so one
// read of the counts covers the plan, the premise and the segments.
extern "C" int ssla_sparse_pool_plan_enqueue(const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w,
                                             const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in,
                                             int B, int H, int W, const int64_t *lut, int64_t n_rf, int A,
                                             int64_t E_cap, void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(G >= 0 && E_in >= 0 && B > 0 && H > 0 && W > 0 && n_rf > 0 && A > 0 && E_cap >= E_in,
                 "sparse_pool_plan: bad arguments");
  SSLA_CHECK_ARG(E_cap < 0x7fffffff && E_in * A < 0x7fffffff,
                 "sparse_pool_plan: the row capacity and E_in * A must stay below 2^31");
  const PoolWs L = pool_layout(workspace, G, B, H, W, n_rf, A, E_cap);
  if (!workspace || workspace_bytes < L.total) {
    set_error("sparse_pool_plan: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the plan with the counting fill's inverse table, without the largest
  // time (only the sort fill needs it)
  // a capacity of one row per event promises one field per pixel (more rows
  // than that are reported at the finish): one thread per event in the fill
  const bool one = E_cap == E_in;
  int s = rf_plan_impl(gr_batch, gr_h, gr_w, gr_len, G, time, E_in, B, H, W, lut, n_rf, A, E_cap, L.inv, one, false,
                       workspace, L.rf.total, st);
  if (s) return s;
  if (E_in > 0) {   // the counting fill, rows bounded by the capacity
    if (one)
      hipLaunchKernelGGL(rf_merge<true>, dim3(grid_for(E_in)), dim3(kThreads), 0, st, L.rf.val, gr_batch, gr_h,
                         gr_w, L.rf.gstart, gr_len, L.rf.pixmap, L.inv, lut, n_rf, A, B, H, W, L.rf.ev_pre, time,
                         E_in, E_cap, L.src, L.tim, static_cast<int64_t *>(nullptr), static_cast<int32_t *>(nullptr),
                         L.rf.act_pre, L.fidx);
    else
      hipLaunchKernelGGL(rf_merge<false>, dim3(grid_for(E_in * A)), dim3(kThreads), 0, st, L.rf.val, gr_batch, gr_h,
                         gr_w, L.rf.gstart, gr_len, L.rf.pixmap, L.inv, lut, n_rf, A, B, H, W, L.rf.ev_pre, time,
                         E_in, E_cap, L.src, L.tim, static_cast<int64_t *>(nullptr), static_cast<int32_t *>(nullptr),
                         L.rf.act_pre, L.fidx);
  }
  s = pool_segments_pass(L, E_cap, st, true);
  if (s) return s;
  return launch_status("sparse_pool_plan");
}

// The plan's counts read back after ssla_sparse_pool_plan_enqueue (head[0..5]
// and bad as ssla_events_counts returns them): checks them and, when a
// pixel run was not sorted by time, runs the sort fill (which reads the
// device twice more).  counts_out as for ssla_sparse_pool_plan.
extern "C" int ssla_sparse_pool_plan_finish(const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in,
                                            int B, int H, int W, const int64_t *lut, int64_t n_rf, int A,
                                            int64_t E_cap, const int64_t *head, int bad, int64_t *counts_out,
                                            void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(G >= 0 && E_in >= 0 && B > 0 && H > 0 && W > 0 && n_rf > 0 && A > 0 && E_cap >= E_in && head &&
                     counts_out,
                 "sparse_pool_plan: bad arguments");
  const int64_t n_f = static_cast<int64_t>(B) * n_rf;
  const PoolWs L = pool_layout(workspace, G, B, H, W, n_rf, A, E_cap);
  if (!workspace || workspace_bytes < L.total) {
    set_error("sparse_pool_plan: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  int64_t c[8] = {};
  for (int i = 0; i < 6; ++i) c[i] = head[i];
  for (int i = 0; i < 4; ++i) counts_out[i] = 0;
  if (bad) {
    counts_out[3] = 1;
    return SSLA_OK;
  }
  if (c[5] != 0) {
    set_error("sparse_pool_plan: a pixel lies in more than one field, but the row capacity (E_cap == E_in) "
              "promises one");
    return SSLA_ERR_ARG;
  }
  const int64_t n_act = c[0], E_out = c[1];
  if (n_act < 0 || n_act > n_f || E_out < 0) {
    set_error("sparse_pool_plan: plan counts outside their bounds");
    return SSLA_ERR_LAUNCH;
  }
  if (E_out > E_cap) {
    set_error("sparse_pool_plan: %lld field rows exceed the capacity %lld", (long long)E_out, (long long)E_cap);
    return SSLA_ERR_ARG;
  }
  int s = SSLA_OK;
  if (c[3] != 0 && E_out > 0) {   // a pixel run not sorted by time: the sort fill
    hipLaunchKernelGGL(max_i64, dim3(grid_for(std::min<int64_t>(E_in, 1 << 16))), dim3(kThreads), 0, st, time, E_in,
                       L.rf.tmax);
    hipLaunchKernelGGL(store_u64_as_i64, dim3(1), dim3(64), 0, st, L.rf.tmax, L.rf.counts + 2);
    s = ssla_events_counts(workspace, c, 5, nullptr, stream);
    if (s) return s;
    const int64_t t_max = c[2];
    if (t_max < 0) {
      set_error("sparse_pool_plan: negative largest time");
      return SSLA_ERR_LAUNCH;
    }
    const uint64_t t_stride = static_cast<uint64_t>(t_max) + 1;
    hipLaunchKernelGGL(rf_enumerate, dim3(grid_for(n_f * A)), dim3(kThreads), 0, st, lut, n_rf, A, B, H, W,
                       L.rf.pixmap, gr_len, L.rf.gstart, L.rf.act, L.rf.act_pre, L.rf.ev_pre, time, E_in, t_stride,
                       L.rf.key, L.rf.val, L.rf.pre_src, L.rf.pre_pos);
    const int end_bit = bits_for(static_cast<uint64_t>(std::max<int64_t>(n_act, 1)) * t_stride);
    s = sort_pairs(L.rf.tmp, L.rf.tmp_bytes, L.rf.key, L.rf.skey, L.rf.val, L.rf.perm, E_out, end_bit, st);
    if (s) return s;
    hipLaunchKernelGGL(rf_emit, dim3(grid_for(E_out)), dim3(kThreads), 0, st, L.rf.perm, E_out, L.rf.pre_src,
                       L.rf.pre_pos, time, L.src, L.tim, static_cast<int64_t *>(nullptr), L.rf.skey, t_stride,
                       L.fidx);
    s = pool_segments_pass(L, E_cap, st, false);
    if (s) return s;
    s = ssla_events_counts(workspace, c, 5, nullptr, stream);
    if (s) return s;
  }
  const int64_t n_seg = c[4];
  if (n_seg < 0 || n_seg > E_out) {
    set_error("sparse_pool_plan: segment count outside its bounds");
    return SSLA_ERR_LAUNCH;
  }
  counts_out[0] = n_act;
  counts_out[1] = n_seg;
  counts_out[2] = E_out;
  return launch_status("sparse_pool_plan");
}

// counts_out[0..3] = active fields, segments, field rows, and 1 if a group
// coordinate or run was out of range (then nothing else was computed):
// the enqueue, one read of the counts, the finish.
extern "C" int ssla_sparse_pool_plan(const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w,
                                     const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in, int B,
                                     int H, int W, const int64_t *lut, int64_t n_rf, int A, int64_t E_cap,
                                     int64_t *counts_out, void *workspace, size_t workspace_bytes, void *stream) {
  SSLA_CHECK_ARG(counts_out, "sparse_pool_plan: bad arguments");
  int s = ssla_sparse_pool_plan_enqueue(gr_batch, gr_h, gr_w, gr_len, G, time, E_in, B, H, W, lut, n_rf, A, E_cap,
                                        workspace, workspace_bytes, stream);
  if (s) return s;
  int64_t c[8] = {};
  int bad = 0;
  s = ssla_events_counts(workspace, c, 6, &bad, stream);
  if (s) return s;
  return ssla_sparse_pool_plan_finish(gr_len, G, time, E_in, B, H, W, lut, n_rf, A, E_cap, c, bad, counts_out,
                                      workspace, workspace_bytes, stream);
}

// After ssla_sparse_pool_plan on the same workspace and sizes: out_events
// [n_seg, C] (mode 0 max, 1 mean), out_time [n_seg], and per active field
// out_len / out_batch / out_h / out_w [n_act]; outcoord is the [n_rf, 2]
// (w, h) output coordinate table of the fields.  The outputs come in two
// parts that may be emitted by separate calls on the same plan: the values
// (out_events; events may then be the only input) and the structure
// (out_time and the per-field outputs); a null out_events skips the values,
// null per-field outputs skip the structure (out_time is then optional).
extern "C" int ssla_sparse_pool_emit(const float *events, int C, int64_t G, int64_t E_in, int B, int H, int W,
                                     int64_t n_rf, int A, int64_t E_cap, const int64_t *outcoord, int mode,
                                     int64_t n_act, int64_t n_seg, int64_t E_out, float *out_events, int64_t *out_time,
                                     int64_t *out_len, int64_t *out_batch, int64_t *out_h, int64_t *out_w,
                                     void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(C > 0 && G >= 0 && E_in >= 0 && B > 0 && H > 0 && W > 0 && n_rf > 0 && A > 0 &&
                     (mode == 0 || mode == 1),
                 "sparse_pool_emit: bad arguments");
  SSLA_CHECK_ARG(E_cap >= E_in && E_cap < 0x7fffffff, "sparse_pool_emit: bad row capacity");
  SSLA_CHECK_ARG(E_out >= 0 && E_out <= E_cap && n_seg >= 0 && n_seg <= E_out && n_act >= 0 &&
                     n_act <= static_cast<int64_t>(B) * n_rf,
                 "sparse_pool_emit: counts outside the plan's bounds");
  const PoolWs L = pool_layout(workspace, G, B, H, W, n_rf, A, E_cap);
  if (!workspace || workspace_bytes < L.total) {
    set_error("sparse_pool_emit: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  const bool values = out_events != nullptr, structure = out_len != nullptr;
  if (!values && !structure) return SSLA_OK;   // nothing requested (or nothing to write: empty outputs)
  SSLA_CHECK_ARG((!values || n_seg == 0 || events) && (!structure || n_seg == 0 || out_time) &&
                     (!structure || n_act == 0 || (outcoord && out_batch && out_h && out_w)),
                 "sparse_pool_emit: null pointer");
  if (E_out * C == 0 && n_act == 0) return SSLA_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  SSLA_CHECK_ARG(E_out * C < 0x7fffffff, "sparse_pool_emit: rows x channels must stay below 2^31");
  const bool vec = C % 4 == 0 && aligned(events, 16) && aligned(out_events, 16);
  const unsigned grid = grid_for(std::max(values ? E_out * (vec ? C / 4 : C) : E_out, n_act));
#define SSLA_POOL_EMIT(MEANV, VWV)                                                                                \
  hipLaunchKernelGGL((pool_emit_rows<MEANV, VWV>), dim3(grid), dim3(kThreads), 0, st, events, E_in, C, L.src,       \
                     L.tim, L.head, L.segx, E_out, n_seg, L.rf.f_index, L.rf.f_len, L.rf.ev_pre, n_act, n_rf,       \
                     outcoord, out_events, out_time, out_len, out_batch, out_h, out_w)
  if (mode == 1) {
    if (vec) SSLA_POOL_EMIT(true, 4);
    else SSLA_POOL_EMIT(true, 1);
  } else {
    if (vec) SSLA_POOL_EMIT(false, 4);
    else SSLA_POOL_EMIT(false, 1);
  }
#undef SSLA_POOL_EMIT
  return launch_status("sparse_pool_emit");
}

extern "C" int ssla_sparse_pool_emit_linear(const float *x, int K, const uint16_t *w, int C, int64_t G, int64_t E_in,
                                            int B, int H, int W, int64_t n_rf, int A, int64_t E_cap, int mode,
                                            int64_t n_act, int64_t n_seg, int64_t E_out, float *out_events,
                                            void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(K == 2, "sparse_pool_emit_linear: K must be 2 (got %d)", K);
  SSLA_CHECK_ARG(C > 0 && C % 4 == 0 && G >= 0 && E_in >= 0 && B > 0 && H > 0 && W > 0 && n_rf > 0 && A > 0 &&
                     (mode == 0 || mode == 1),
                 "sparse_pool_emit_linear: bad arguments (C must be a multiple of 4)");
  SSLA_CHECK_ARG(E_cap >= E_in && E_cap < 0x7fffffff, "sparse_pool_emit_linear: bad row capacity");
  SSLA_CHECK_ARG(E_out >= 0 && E_out <= E_cap && n_seg >= 0 && n_seg <= E_out && n_act >= 0 &&
                     n_act <= static_cast<int64_t>(B) * n_rf,
                 "sparse_pool_emit_linear: counts outside the plan's bounds");
  const PoolWs L = pool_layout(workspace, G, B, H, W, n_rf, A, E_cap);
  if (!workspace || workspace_bytes < L.total) {
    set_error("sparse_pool_emit_linear: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  if (E_out == 0 || n_seg == 0) return SSLA_OK;
  SSLA_CHECK_ARG(x && w && out_events, "sparse_pool_emit_linear: null pointer");
  SSLA_CHECK_ARG(aligned(x, 8) && aligned(out_events, 16), "sparse_pool_emit_linear: x must be 8-byte and "
                 "out_events 16-byte aligned");
  SSLA_CHECK_ARG(E_out * C < 0x7fffffff, "sparse_pool_emit_linear: rows x channels must stay below 2^31");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(E_out * (C / 4));
  if (mode == 1)
    hipLaunchKernelGGL((pool_emit_rows<true, 4, true>), dim3(grid), dim3(kThreads), 0, st, x, E_in, C, L.src, L.tim,
                       L.head, L.segx, E_out, n_seg, L.rf.f_index, L.rf.f_len, L.rf.ev_pre, (int64_t)0, n_rf,
                       static_cast<const int64_t *>(nullptr), out_events, static_cast<int64_t *>(nullptr),
                       static_cast<int64_t *>(nullptr), static_cast<int64_t *>(nullptr),
                       static_cast<int64_t *>(nullptr), static_cast<int64_t *>(nullptr), w);
  else
    hipLaunchKernelGGL((pool_emit_rows<false, 4, true>), dim3(grid), dim3(kThreads), 0, st, x, E_in, C, L.src, L.tim,
                       L.head, L.segx, E_out, n_seg, L.rf.f_index, L.rf.f_len, L.rf.ev_pre, (int64_t)0, n_rf,
                       static_cast<const int64_t *>(nullptr), out_events, static_cast<int64_t *>(nullptr),
                       static_cast<int64_t *>(nullptr), static_cast<int64_t *>(nullptr),
                       static_cast<int64_t *>(nullptr), static_cast<int64_t *>(nullptr), w);
  return launch_status("sparse_pool_emit_linear");
}

// ---- rows ------------------------------------------------------------------------
extern "C" int ssla_gather_rows(const float *src, int64_t n_src, const int64_t *idx, int64_t m, int C, float *out,
                                void *stream) {
  clear_error();
  SSLA_CHECK_ARG(n_src >= 0 && m >= 0 && C > 0, "gather_rows: bad sizes");
  if (m == 0) return SSLA_OK;
  SSLA_CHECK_ARG(src && idx && out, "gather_rows: null pointer");
  hipLaunchKernelGGL(gather_rows_kernel, dim3(grid_for(m * C)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     src, idx, m, n_src, C, out);
  return launch_status("gather_rows");
}

namespace {
struct IaWs {
  uint64_t *key, *skey;
  int32_t *val, *perm, *bad;
  void *tmp;
  size_t tmp_bytes, total;
};
IaWs ia_layout(void *ws, int64_t n) {
  Carve c{static_cast<char *>(ws)};
  IaWs L;
  c.take<int64_t>(8);   // counts slot (unused here)
  L.bad = c.take<int32_t>(8);
  L.key = c.take<uint64_t>(n);
  L.skey = c.take<uint64_t>(n);
  L.val = c.take<int32_t>(n);
  L.perm = c.take<int32_t>(n);
  L.tmp_bytes = sort_temp_bytes(n);
  L.tmp = c.take<char>(L.tmp_bytes);
  L.total = c.off;
  return L;
}
}  // namespace

extern "C" size_t ssla_index_add_rows_workspace_size(int64_t n) {
  return n < 0 ? 0 : ia_layout(nullptr, n).total;
}

extern "C" int ssla_index_add_rows(const float *src, const int64_t *idx, int64_t n, int C, int64_t n_out, float *out,
                                   void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(n >= 0 && C > 0 && n_out >= 0 && n < 0x7fffffff, "index_add_rows: bad sizes");
  const IaWs L = ia_layout(workspace, n);
  if (!workspace || workspace_bytes < L.total) {
    set_error("index_add_rows: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_i32, dim3(1), dim3(kThreads), 0, st, L.bad, (int64_t)8, 0);
  if (n_out == 0) return launch_status("index_add_rows");
  SSLA_CHECK_ARG(out && (n == 0 || (src && idx)), "index_add_rows: null pointer");
  if (n > 0) {
    hipLaunchKernelGGL(idx_keys, dim3(grid_for(n)), dim3(kThreads), 0, st, idx, n, n_out, L.key, L.val, L.bad);
    const int s = sort_pairs(L.tmp, L.tmp_bytes, L.key, L.skey, L.val, L.perm, n, bits_for(n_out), st);
    if (s) return s;
  }
  hipLaunchKernelGGL(index_add_rows, dim3(static_cast<unsigned>((n_out + 3) / 4)), dim3(256), 0, st, src, L.skey,
                     L.perm, n, n_out, C, out);
  return launch_status("index_add_rows");
}

// ---- stable sort of (uint64 key, int32 value) pairs --------------------------------
extern "C" size_t ssla_sort_pairs_workspace_size(int64_t n) {
  return n < 0 ? 0 : align256(sort_temp_bytes(n)) + align256(sizeof(int32_t) * std::max<int64_t>(n, 1));
}

// vals_in may be NULL (then the values are 0..n-1).  end_bit: number of
// low key bits that take part (1..64).
extern "C" int ssla_sort_pairs(const uint64_t *keys_in, const int32_t *vals_in, int64_t n, int end_bit,
                               uint64_t *keys_out, int32_t *vals_out, void *workspace, size_t workspace_bytes,
                               void *stream) {
  clear_error();
  SSLA_CHECK_ARG(n >= 0 && n < 0x7fffffff && end_bit >= 1 && end_bit <= 64, "sort_pairs: bad arguments");
  const size_t need = ssla_sort_pairs_workspace_size(n);
  if (!workspace || workspace_bytes < need) {
    set_error("sort_pairs: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  if (n == 0) return SSLA_OK;
  SSLA_CHECK_ARG(keys_in && keys_out && vals_out, "sort_pairs: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t tb = sort_temp_bytes(n);
  const int32_t *vin = vals_in;
  if (!vin) {
    int32_t *iota = reinterpret_cast<int32_t *>(static_cast<char *>(workspace) + align256(tb));
    hipLaunchKernelGGL(iota_i32, dim3(grid_for(n)), dim3(kThreads), 0, st, iota, n);
    vin = iota;
  }
  const int s = sort_pairs(workspace, tb, keys_in, keys_out, vin, vals_out, n, end_bit, st);
  if (s) return s;
  return launch_status("sort_pairs");
}

// ---- segments ---------------------------------------------------------------------
namespace {
struct SegWs {
  int64_t *counts, *start, *kl, *kpre;
  int32_t *bad;
  void *tmp;
  size_t tmp_bytes, total;
};
SegWs seg_layout(void *ws, int64_t n_seq) {
  Carve c{static_cast<char *>(ws)};
  SegWs L;
  L.counts = c.take<int64_t>(8);
  L.bad = c.take<int32_t>(8);
  L.start = c.take<int64_t>(n_seq + 1);
  L.kl = c.take<int64_t>(n_seq + 1);
  L.kpre = c.take<int64_t>(n_seq + 1);
  L.tmp_bytes = scan_temp_bytes(n_seq + 1);
  L.tmp = c.take<char>(L.tmp_bytes);
  L.total = c.off;
  return L;
}
}  // namespace

extern "C" size_t ssla_segments_workspace_size(int64_t n_seq) {
  return n_seq < 0 ? 0 : seg_layout(nullptr, n_seq).total;
}

// truncate_packed_sequence: keep the first `threshold` rows of every
// sequence of data [E, C] (and of others [E], when given).  counts[0] = rows
// kept.  out_data / out_others hold E rows of capacity.
extern "C" int ssla_truncate_packed(const float *data, const int64_t *seqlens, int64_t n_seq, int64_t E, int C,
                                    int64_t threshold, const int64_t *others, float *out_data, int64_t *out_lengths,
                                    int64_t *out_others, void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && E >= 0 && C > 0 && threshold >= 0, "truncate_packed: bad sizes");
  const SegWs L = seg_layout(workspace, n_seq);
  if (!workspace || workspace_bytes < L.total) {
    set_error("truncate_packed: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_i64, dim3(1), dim3(kThreads), 0, st, L.counts, (int64_t)8, (int64_t)0);
  if (n_seq == 0) return launch_status("truncate_packed");
  SSLA_CHECK_ARG(seqlens && out_lengths && (E == 0 || (data && out_data)) && (!others || out_others),
                 "truncate_packed: null pointer");
  int s = excl_scan(L.tmp, L.tmp_bytes, seqlens, L.start, n_seq, st);
  if (s) return s;
  hipLaunchKernelGGL(trunc_len, dim3(grid_for(n_seq)), dim3(kThreads), 0, st, seqlens, n_seq, threshold, L.kl);
  s = excl_scan(L.tmp, L.tmp_bytes, L.kl, L.kpre, n_seq, st);
  if (s) return s;
  hipLaunchKernelGGL(total_from_scan, dim3(1), dim3(64), 0, st, L.kpre, L.kl, n_seq, L.counts);
  if (E > 0)
    hipLaunchKernelGGL(trunc_copy, dim3(grid_for(n_seq)), dim3(kThreads), 0, st, data, others, L.start, L.kl, L.kpre,
                       n_seq, E, C, out_data, out_others);
  if (hipMemcpyAsync(out_lengths, L.kl, sizeof(int64_t) * n_seq, hipMemcpyDeviceToDevice, st) != hipSuccess) {
    set_error("truncate_packed: copy of the lengths failed");
    return SSLA_ERR_LAUNCH;
  }
  return launch_status("truncate_packed");
}

// TemporalDropout keep indices: per sequence ceil(len / w) indices, every
// w-th row, aligned so that the last row is kept.  counts[0] = kept rows;
// out_idx holds idx_cap rows, and a count above idx_cap means the rows past
// it were not written.
extern "C" int ssla_temporal_dropout_index(const int64_t *lengths, int64_t n_seq, int64_t window, int64_t *out_idx,
                                           int64_t idx_cap, int64_t *out_lengths, void *workspace,
                                           size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && window > 0 && idx_cap >= 0, "temporal_dropout_index: bad arguments");
  const SegWs L = seg_layout(workspace, n_seq);
  if (!workspace || workspace_bytes < L.total) {
    set_error("temporal_dropout_index: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_i64, dim3(1), dim3(kThreads), 0, st, L.counts, (int64_t)8, (int64_t)0);
  if (n_seq == 0) return launch_status("temporal_dropout_index");
  SSLA_CHECK_ARG(lengths && out_idx && out_lengths, "temporal_dropout_index: null pointer");
  int s = excl_scan(L.tmp, L.tmp_bytes, lengths, L.start, n_seq, st);
  if (s) return s;
  hipLaunchKernelGGL(td_len, dim3(grid_for(n_seq)), dim3(kThreads), 0, st, lengths, n_seq, window, L.kl);
  s = excl_scan(L.tmp, L.tmp_bytes, L.kl, L.kpre, n_seq, st);
  if (s) return s;
  hipLaunchKernelGGL(total_from_scan, dim3(1), dim3(64), 0, st, L.kpre, L.kl, n_seq, L.counts);
  hipLaunchKernelGGL(td_index, dim3(grid_for(n_seq)), dim3(kThreads), 0, st, lengths, L.start, L.kl, L.kpre, n_seq,
                     window, idx_cap, out_idx);
  if (hipMemcpyAsync(out_lengths, L.kl, sizeof(int64_t) * n_seq, hipMemcpyDeviceToDevice, st) != hipSuccess) {
    set_error("temporal_dropout_index: copy of the lengths failed");
    return SSLA_ERR_LAUNCH;
  }
  return launch_status("temporal_dropout_index");
}

// out[i] = values[s] for every element i of segment s (repeat_interleave);
// n = sum of lengths (elements beyond the segments are left untouched).
extern "C" int ssla_expand_segments(const int64_t *values, const int64_t *lengths, int64_t n_seq, int64_t n,
                                    int64_t *out, void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && n >= 0, "expand_segments: bad sizes");
  const SegWs L = seg_layout(workspace, n_seq);
  if (!workspace || workspace_bytes < L.total) {
    set_error("expand_segments: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  if (n_seq == 0 || n == 0) return SSLA_OK;
  SSLA_CHECK_ARG(values && lengths && out, "expand_segments: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int s = excl_scan(L.tmp, L.tmp_bytes, lengths, L.start, n_seq, st);
  if (s) return s;
  hipLaunchKernelGGL(expand_segments, dim3(grid_for(n_seq)), dim3(kThreads), 0, st, values, L.start, lengths, n_seq, n,
                     out);
  return launch_status("expand_segments");
}

// SparsePool keys: events of field f (fields in order, lengths[f] each)
// with equal time form one pooling segment.  seg[i] = segment of event i
// (non-decreasing: the sorted index the pooling kernels take), seg_time /
// seg_field per segment, new_lengths[f] = segments of field f.
// counts[0] = segments.  field[i] (the field of event i) is scratch [E].
extern "C" int ssla_pool_segments(const int64_t *time, const int64_t *lengths, int64_t n_f, int64_t E, int64_t *field,
                                  int64_t *seg, int64_t *seg_time, int64_t *seg_field, int64_t *new_lengths,
                                  void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(n_f >= 0 && E >= 0, "pool_segments: bad sizes");
  const SegWs L = seg_layout(workspace, std::max(n_f, E));
  if (!workspace || workspace_bytes < L.total) {
    set_error("pool_segments: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_i64, dim3(1), dim3(kThreads), 0, st, L.counts, (int64_t)8, (int64_t)0);
  if (n_f == 0) return launch_status("pool_segments");
  SSLA_CHECK_ARG(lengths && new_lengths && (E == 0 || (time && field && seg && seg_time && seg_field)),
                 "pool_segments: null pointer");
  hipLaunchKernelGGL(fill_i64, dim3(grid_for(n_f)), dim3(kThreads), 0, st, new_lengths, n_f, (int64_t)0);
  if (E == 0) return launch_status("pool_segments");
  // field of every event (repeat_interleave of 0..n_f-1)
  int s = excl_scan(L.tmp, L.tmp_bytes, lengths, L.start, n_f, st);
  if (s) return s;
  hipLaunchKernelGGL(pool_field_of, dim3(grid_for(E)), dim3(kThreads), 0, st, L.start, lengths, n_f, E, field);
  // segment heads and their prefix
  int64_t *head = L.kl;   // layout holds max(n_f, E) + 1 entries
  hipLaunchKernelGGL(pool_heads, dim3(grid_for(E)), dim3(kThreads), 0, st, time, field, E, head);
  s = excl_scan(L.tmp, L.tmp_bytes, head, L.kpre, E, st);
  if (s) return s;
  hipLaunchKernelGGL(total_from_scan, dim3(1), dim3(64), 0, st, L.kpre, head, E, L.counts);
  hipLaunchKernelGGL(pool_emit, dim3(grid_for(E)), dim3(kThreads), 0, st, head, L.kpre, time, field, E, seg, seg_time,
                     seg_field);
  hipLaunchKernelGGL(count_sorted_by, dim3(grid_for(n_f)), dim3(kThreads), 0, st, seg_field, L.counts, 0, n_f,
                     new_lengths);
  return launch_status("pool_segments");
}

// Sparse-to-dense grid: the last event of every group at its (b, h, w) cell
// of grid [B, C, Hg, Wg] (other cells untouched; the caller zeroes the grid).
extern "C" int ssla_events_to_grid(const float *events, int64_t E, int C, const int64_t *lengths,
                                   const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w, int64_t G, int B,
                                   int Hg, int Wg, float *grid, void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(E >= 0 && C > 0 && G >= 0 && B > 0 && Hg > 0 && Wg > 0, "events_to_grid: bad sizes");
  const SegWs L = seg_layout(workspace, G);
  if (!workspace || workspace_bytes < L.total) {
    set_error("events_to_grid: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_i32, dim3(1), dim3(kThreads), 0, st, L.bad, (int64_t)8, 0);
  if (G == 0) return launch_status("events_to_grid");
  SSLA_CHECK_ARG(events && lengths && gr_batch && gr_h && gr_w && grid, "events_to_grid: null pointer");
  // end of every group = inclusive prefix of lengths
  int s = excl_scan(L.tmp, L.tmp_bytes, lengths, L.start, G, st);
  if (s) return s;
  hipLaunchKernelGGL(seg_ends, dim3(grid_for(G)), dim3(kThreads), 0, st, L.start, lengths, G, L.kl);
  hipLaunchKernelGGL(grid_place, dim3(grid_for(G * C)), dim3(kThreads), 0, st, events, L.kl, gr_batch, gr_h, gr_w, G,
                     E, C, B, Hg, Wg, grid, L.bad);
  return launch_status("events_to_grid");
}

extern "C" int ssla_events_to_grids(const ssla_grid_level *levels, int n_levels, int B, int32_t *status,
                                    void *stream) {
  clear_error();
  SSLA_CHECK_ARG(levels && n_levels > 0 && n_levels <= SSLA_GRIDS_MAX_LEVELS && B > 0,
                 "events_to_grids: bad arguments (levels=%d B=%d)", n_levels, B);
  GridArgs a{};
  a.n_levels = n_levels;
  a.B = B;
  int blocks = 0;
  int64_t max_cells = 1;
  for (int l = 0; l < n_levels; ++l) {
    const ssla_grid_level &lv = levels[l];
    SSLA_CHECK_ARG(lv.E >= 0 && lv.G >= 0 && lv.C > 0 && lv.Hg > 0 && lv.Wg > 0 && lv.grid,
                   "events_to_grids: bad level %d", l);
    SSLA_CHECK_ARG(lv.G == 0 || (lv.events && lv.lengths && lv.batch && lv.h && lv.w),
                   "events_to_grids: null pointer in level %d", l);
    SSLA_CHECK_ARG(lv.E < 0x7fffffff, "events_to_grids: level %d has 2^31 events or more", l);
    const int64_t cells = static_cast<int64_t>(B) * lv.Hg * lv.Wg;
    if (cells > SSLA_GRIDS_MAX_CELLS) {
      set_error("events_to_grids: level %d has %lld cells (at most %d)", l, static_cast<long long>(cells),
                SSLA_GRIDS_MAX_CELLS);
      return SSLA_ERR_UNSUPPORTED;
    }
    a.lv[l] = lv;
    a.blk0[l] = blocks;
    blocks += (lv.C + kGridCB - 1) / kGridCB;
    SSLA_CHECK_ARG(blocks < (1 << 20), "events_to_grids: too many channels");
    max_cells = std::max(max_cells, cells);
  }
  a.blk0[n_levels] = blocks;
  hipLaunchKernelGGL(grids_kernel, dim3(blocks), dim3(kGridThreads), static_cast<size_t>(max_cells) * sizeof(int32_t),
                     static_cast<hipStream_t>(stream), a, status);
  return launch_status("events_to_grids");
}

// Per-pixel delays in place (MosModel.preprocess_inputs, model_mos.py:195-201):
// column 0 of feat [E, C] (timestamps) becomes min((t_i - t_{i-1}) / 1e5, 1)
// within every group and 1 at the first event of a group.
extern "C" int ssla_pixel_delays(float *feat, int64_t E, int C, const int64_t *lengths, int64_t G, void *workspace,
                                 size_t workspace_bytes, void *stream) {
  clear_error();
  SSLA_CHECK_ARG(E >= 0 && C > 0 && G >= 0, "pixel_delays: bad sizes");
  const SegWs L = seg_layout(workspace, G);
  if (!workspace || workspace_bytes < L.total) {
    set_error("pixel_delays: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  if (G == 0 || E == 0) return SSLA_OK;
  SSLA_CHECK_ARG(feat && lengths, "pixel_delays: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int s = excl_scan(L.tmp, L.tmp_bytes, lengths, L.start, G, st);
  if (s) return s;
  hipLaunchKernelGGL(pixel_delays, dim3(grid_for(G)), dim3(kThreads), 0, st, feat, L.start, lengths, G, E, C);
  return launch_status("pixel_delays");
}
