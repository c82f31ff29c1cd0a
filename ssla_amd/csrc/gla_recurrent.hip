// Fused recurrent GLA forward (serial over time, state in registers).
//
// Semantics follow naive_gla_recurrent (reference ops/gla/naive.py:50-111):
//   S_t = exp(g_t)[:, None] * S_{t-1} + k_t v_t^T,   o_t = (scale q_t) . S_t
// with the initial state taken from h0 (or zero) and the final state written
// to ht.  One wavefront owns one (sequence, head, 16-column V tile); its 64
// lanes are 4 key-groups x 16 value columns, each lane holding KPL rows of
// the fp32 state.  The o reduction over the 4 key-groups is two xor-shuffles.
#include <utility>

#include "common.h"

namespace ssla {
namespace {

#ifndef SSLA_GR_WPB
#define SSLA_GR_WPB 4
#endif
// wavefronts (units) per workgroup of the staged recurrence kernels
constexpr int kRecWaves = SSLA_GR_WPB;

constexpr int kBV = 16;   // value columns per wavefront
constexpr int kKG = 4;    // key groups per wavefront (64 / kBV)

// A sequence whose state row is outside [0, n_rows) or not above the row of
// the sequence before it (state_idx must be strictly increasing, so no two
// sequences share a state row) is skipped: its o rows are written as zeros,
// no state is read or written, and the status word is set to SSLA_ERR_ARG.
__device__ __forceinline__ bool bad_state_row(const int32_t *state_idx, int n, int64_t srow, int n_rows) {
  return state_idx && (srow < 0 || srow >= n_rows || (n > 0 && static_cast<int64_t>(state_idx[n - 1]) >= srow));
}

template <int DT>
__device__ __forceinline__ void skip_sequence(void *o, int64_t bos, int64_t eos, int H, int h, int V, int col,
                                              bool writer, int lane, int32_t *status) {
  if (writer)
    for (int64_t t = bos; t < eos; ++t) Elem<DT>::store(o, (t * H + h) * V + col, 0.f);
  if (status && lane == 0) __hip_atomic_store(status, SSLA_ERR_ARG, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------- staged kernel --
// Each wavefront owns one unit: (sequence, head, 16-column V tile), or a
// segment of a sequence in the segmented schedule; its lanes are 4 key
// groups x 16 value columns, each lane holding KPL = K/4 fp32 state rows.
// A unit is walked in blocks of kSB steps: a block's q, k, g rows (this
// head) and v tile are fetched with 16-byte buffer loads into registers
// while the previous block is being computed, then parked in a wave-private LDS buffer, from which every step reads its
// KPL keys (the 16 lanes of a key group read the same address: one
// broadcast).  A sequence of n steps therefore waits on about n / kSB
// memory round trips instead of n.  The decays exp(g) of a block are
// computed once per (step, key) while the block is parked (fp32 in LDS),
// not once per value column, and the output scale is applied once to the
// reduced dot product.  Rows past the sequence end fall outside the block's
// buffer resources and read as zeros (decay 1 and k = 0 leave the state
// unchanged), and their outputs are not stored.
constexpr int kSB = 16;   // steps per staged block
constexpr int kFoldB = 2; // segment states folded per round trip

template <int DT, int GDT, int KPL>
struct Staged {
  static constexpr int K = 4 * KPL;
  static constexpr int ES = DT == SSLA_F32 ? 4 : 2;    // bytes per q/k/v element
  static constexpr int GS = GDT == SSLA_F32 ? 4 : 2;   // bytes per g element
  static constexpr int QB = K * ES, GB = K * GS, VB = kBV * ES;   // row bytes (v: one tile)
  static constexpr int PQ = kSB * QB / 16, PG = kSB * GB / 16, PV = kSB * VB / 16;   // 16-byte pieces
  static constexpr int NQ = (PQ + 63) / 64, NG = (PG + 63) / 64, NV = (PV + 63) / 64;
  static constexpr int DB = K * 4;            // bytes of a row of fp32 decays, and of parked q / k rows
  static constexpr int OQ = 0, OK = kSB * DB, OD = 2 * kSB * DB, OV = 3 * kSB * DB;
  static constexpr int BYTES = OV + kSB * VB;   // LDS per wavefront
};

constexpr uint32_t kNoRow = 0x80000000u;   // an offset past every resource: reads zeros
constexpr int kRawRsrc = 0x00020000;        // raw 32-bit data, range checked

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void *base, int64_t bytes) {
  bytes = min(bytes, static_cast<int64_t>(0x7ffffff0));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), kRawRsrc);
}

// N (4, 8 or 16) consecutive elements of type DT at byte address p of LDS.
template <int DT, int N>
__device__ __forceinline__ void lds_run(const unsigned char *p, float (&x)[N]) {
  if constexpr (DT == SSLA_F32) {
#pragma unroll
    for (int j = 0; j < N / 4; ++j) {
      const float4 t = *reinterpret_cast<const float4 *>(p + 16 * j);
      x[4 * j] = t.x; x[4 * j + 1] = t.y; x[4 * j + 2] = t.z; x[4 * j + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N / 4; ++j) {
      const uint2 u = *reinterpret_cast<const uint2 *>(p + 8 * j);
      const uint16_t e[4] = {static_cast<uint16_t>(u.x), static_cast<uint16_t>(u.x >> 16),
                             static_cast<uint16_t>(u.y), static_cast<uint16_t>(u.y >> 16)};
#pragma unroll
      for (int c = 0; c < 4; ++c) x[4 * j + c] = DT == SSLA_BF16 ? bf16_bits_to_f32(e[c]) : f16_bits_to_f32(e[c]);
    }
  }
}

template <int DT>
__device__ __forceinline__ float lds_elem(const unsigned char *p) {
  if constexpr (DT == SSLA_F32) return *reinterpret_cast<const float *>(p);
  else {
    const uint16_t b = *reinterpret_cast<const uint16_t *>(p);
    return DT == SSLA_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
  }
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------- segmented schedule --
// Long sequences are cut into segments of seg_steps steps (kSegSteps,
// halved down to kSegStepsMin while the grid would hold fewer than
// kSegUnits wavefronts; at least one segment per sequence, so empty
// sequences still pass h0 to ht), numbered globally
// (segoff[n] = first segment of sequence n, computed on the device).
// * state pass (kSegState): every segment but the last of its sequence runs
//   from a zero state and leaves its local end state L_j and the product
//   P_j of its decays (per key); the first segment also copies h0 (read
//   once, here) into the workspace.
// * output pass (kSegOut): segment s of a sequence enters with
//   E = h0, E = P_j E + L_j for j < s (the recurrence is linear in the
//   state, so this is the state after segment s - 1 up to rounding), runs its
//   steps writing o, and the last segment writes ht.  Multi-segment
//   sequences read h0 from the copy, so an in-place update (ht == h0) never
//   races with a segment that has not read it yet.
#ifndef SSLA_REC_SEG_STEPS
#define SSLA_REC_SEG_STEPS 128
#endif
#ifndef SSLA_REC_SEG_MIN
#define SSLA_REC_SEG_MIN 32
#endif
#ifndef SSLA_REC_SEG_UNITS
#define SSLA_REC_SEG_UNITS 8192
#endif
#ifndef SSLA_REC_SEG_FOLD
#define SSLA_REC_SEG_FOLD 8
#endif
constexpr int kSegSteps = SSLA_REC_SEG_STEPS;   // the longest segment
constexpr int kSegStepsMin = SSLA_REC_SEG_MIN;
constexpr int64_t kSegUnits = SSLA_REC_SEG_UNITS;   // wavefront units the segment length aims at (8 per SIMD)
constexpr int64_t kSegFoldMax = SSLA_REC_SEG_FOLD;  // average segments per sequence at most, when halving
#ifndef SSLA_REC_SEG_AVG
#define SSLA_REC_SEG_AVG (SSLA_REC_SEG_STEPS / 2)
#endif
// average steps per sequence below which one pass runs: at the C5 step's
// stage 2 (1,140 sites, 44 events each on average) one pass takes 83-87 µs,
// segments of up to 128 (or 64) steps 102-103 (89-91)
constexpr int64_t kSegAvgMin = SSLA_REC_SEG_AVG;
enum { kPlain = 0, kSegState = 1, kSegOut = 2 };

struct SegWs {
  const int64_t *segoff;   // [n_seq + 1]
  const int4 *segmap;      // [n_segs_max]: (sequence, segment of it, its segment count, 0)
  float *slot;             // [n_segs_max, H, K, V]: L_j
  float *prod;             // [n_segs_max, H, K]: P_j
  float *h0c;              // [n_seq, H, K, V]: copy of the initial states
  int64_t n_segs_max;      // upper bound of the segment count (grid size)
  int seg_steps;           // steps per segment (the last of a sequence may be shorter)
};

// segoff[n] = segments of sequences 0..n-1 (segoff[n_seq]: the total) and
// segmap[s] = (sequence, segment of it, its segment count) for every
// segment s below the total.  One workgroup of 256 threads.  The grid holds n_segs_max segments, which
// bounds the total when cu_seqlens is non-decreasing (the sequences then
// share the T rows); with sequences that overlap the total can exceed it,
// and the segments past the grid would not run: the total is then capped at
// n_segs_max and SSLA_ERR_ARG goes to the status word (when one is given).
__global__ __launch_bounds__(256) void seg_offsets_kernel(const int64_t *__restrict__ cu, int n_seq, int64_t T,
                                                          int seg_steps, int64_t n_segs_max,
                                                          int64_t *__restrict__ segoff, int4 *__restrict__ segmap,
                                                          int32_t *__restrict__ status) {
  __shared__ int64_t ps[256];
  int64_t carry = 0;
  for (int base = 0; base < n_seq; base += 256) {
    const int n = base + static_cast<int>(threadIdx.x);
    int64_t c = 0;
    if (n < n_seq) {
      const int64_t bos = min(max(cu[n], (int64_t)0), T);
      const int64_t eos = min(max(cu[n + 1], bos), T);
      c = max((eos - bos + seg_steps - 1) / seg_steps, (int64_t)1);
    }
    ps[threadIdx.x] = c;
    __syncthreads();
    for (int d = 1; d < 256; d <<= 1) {   // inclusive scan (Hillis-Steele)
      const int64_t x = threadIdx.x >= static_cast<unsigned>(d) ? ps[threadIdx.x - d] : 0;
      __syncthreads();
      ps[threadIdx.x] += x;
      __syncthreads();
    }
    if (n < n_seq) {
      const int64_t first = carry + ps[threadIdx.x] - c;
      segoff[n] = min(first, n_segs_max);
      // each segment's sequence and place in it, so a wavefront finds its
      // unit with one load instead of a search over segoff
      for (int64_t j = 0; j < c && first + j < n_segs_max; ++j)
        segmap[first + j] = make_int4(n, static_cast<int>(j), static_cast<int>(c), 0);
    }
    carry += ps[255];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    segoff[n_seq] = min(carry, n_segs_max);
    if (carry > n_segs_max && status != nullptr) *status = SSLA_ERR_ARG;
  }
}

// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile
// time (the index is a constant expression inside f).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Four values summed over the four 16-lane rows (key groups) at once, row r
// receiving the total of value r: v_permlane16_swap(a, b) swaps a's odd rows
// with b's even rows, so a + b then holds (a0 + a1, b0 + b1, a2 + a3,
// b2 + b3) by row; v_permlane32_swap of two such sums puts the row pairs
// side by side.  VALU lane swaps, no LDS; three swaps and three adds for
// four values, each summed as (x0 + x1) + (x2 + x3).
__device__ __forceinline__ float sum4_key_groups(float a, float b, float c, float d) {
  const u32x2 p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const u32x2 q = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(d), false, false);
  const float ab = __uint_as_float(p.x) + __uint_as_float(p.y);   // rows: a01, b01, a23, b23
  const float cd = __uint_as_float(q.x) + __uint_as_float(q.y);   // rows: c01, d01, c23, d23
  const u32x2 r = __builtin_amdgcn_permlane32_swap(__float_as_uint(ab), __float_as_uint(cd), false, false);
  return __uint_as_float(r.x) + __uint_as_float(r.y);             // rows: a, b, c, d
}

// One output element, rounded to nearest even by the conversion
// instructions (no branches).
// (rs: the rows' buffer resource, off: this lane's byte offset; stores
// past the resource's end are dropped by the hardware range check)
template <int DT>
__device__ __forceinline__ void store_out(__amdgpu_buffer_rsrc_t rs, uint32_t off, float x) {
  if constexpr (DT == SSLA_BF16) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, static_cast<__bf16>(x)), rs, off, 0, 0);
  } else if constexpr (DT == SSLA_F16) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, static_cast<_Float16>(x)), rs, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), rs, off, 0, 0);
  }
}

// One unit of work of a wavefront: (sequence or segment, head, V tile).
struct Unit {
  int64_t bos, eos;   // this unit's steps
  int srow;           // state row of the sequence
  int gseg;           // global segment index (segmented modes)
  int seg, nseg;      // segment of its sequence, segments of the sequence
  int n, h, vt;
  bool run;           // steps to run (false: past the unit count, or nothing to do in this mode)
  bool bad;           // state row outside the table or out of order: skipped, reported
};

template <int DT, int GDT, int KPL, int MODE>
__global__ __launch_bounds__(64 * kRecWaves, (KPL <= 8 ? 4 : 3) * 4 / kRecWaves) void gla_recurrent_staged_kernel(
    const void *__restrict__ q, const void *__restrict__ k,
    const void *__restrict__ v, const void *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int H, int V,
    float scale, const float *__restrict__ h0, void *__restrict__ o,
    float *__restrict__ ht, const int32_t *__restrict__ state_idx, int n_state_rows,
    int64_t T, int32_t *__restrict__ status, SegWs sw) {
  typedef Staged<DT, GDT, KPL> G;
  constexpr int K = G::K;
  __shared__ __align__(16) unsigned char smem[kRecWaves][G::BYTES];
  const int lane = threadIdx.x & 63;
  // wavefront-uniform (SGPR): the unit indexing below runs on the scalar unit
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  unsigned char *lds = smem[wv];
  const int n_vt = (V + kBV - 1) / kBV;
  // items (unit, head, V tile) fit in 31 bits (checked by the host)
  const int n_units = MODE == kPlain ? n_seq : static_cast<int>(sw.n_segs_max);
  const int n_items = n_units * H * n_vt;
  const int kg = lane >> 4;
  const int k0 = kg * KPL;

  auto unit_at = [&](int item) __attribute__((always_inline)) {
    Unit u{};
    u.run = false;
    u.bad = false;
    if (item >= n_items) return u;
    u.vt = item % n_vt;
    u.h = (item / n_vt) % H;
    const int un = item / (n_vt * H);   // sequence, or global segment
    u.n = un;
    u.gseg = un;
    u.seg = 0;
    u.nseg = 1;
    if (MODE != kPlain) {
      const int64_t n_segs = sw.segoff[n_seq];
      const int4 m = sw.segmap[un];   // written for every segment below n_segs
      if (un >= n_segs) return u;     // past the actual segment count
      u.n = m.x;
      u.seg = m.y;
      u.nseg = m.z;
      if (MODE == kSegState && u.seg == u.nseg - 1) return u;   // the last segment needs no local state
    }
    const int64_t sbos = min(max(cu_seqlens[u.n], (int64_t)0), T);
    const int64_t seos = min(max(cu_seqlens[u.n + 1], sbos), T);
    u.bos = MODE == kPlain ? sbos : min(sbos + static_cast<int64_t>(u.seg) * sw.seg_steps, seos);
    u.eos = MODE == kPlain ? seos : min(u.bos + sw.seg_steps, seos);
    u.srow = state_idx ? state_idx[u.n] : u.n;
    u.bad = bad_state_row(state_idx, u.n, u.srow, n_state_rows);
    u.run = !u.bad;
    return u;
  };
  auto col_of = [&](const Unit &u) __attribute__((always_inline)) { return u.vt * kBV + (lane & 15); };
  auto elem0 = [&](const Unit &u) __attribute__((always_inline)) {   // this lane's element (i = 0) of a state
    return (static_cast<int64_t>(u.h) * K + k0) * V + col_of(u);
  };

  // The state a unit starts from: h0 (or its copy) for a whole sequence or a
  // first segment, zero for a state-pass segment.  The first state-pass
  // segment of a sequence also copies h0 into the workspace.
  auto init_state = [&](const Unit &u, float (&S)[KPL]) __attribute__((always_inline)) {
    const bool col_ok = col_of(u) < V;
    const int64_t e0 = elem0(u);
    if (MODE == kSegState) {
#pragma unroll
      for (int i = 0; i < KPL; ++i) S[i] = 0.f;
      if (u.seg == 0 && col_ok) {
        float *dst = sw.h0c + static_cast<int64_t>(u.n) * H * K * V + e0;
#pragma unroll
        for (int i = 0; i < KPL; ++i) dst[i * V] = h0 ? h0[static_cast<int64_t>(u.srow) * H * K * V + e0 + i * V] : 0.f;
      }
    } else {
      const float *src = nullptr;
      if (MODE == kSegOut && u.nseg > 1) src = sw.h0c + static_cast<int64_t>(u.n) * H * K * V;
      else if (h0) src = h0 + static_cast<int64_t>(u.srow) * H * K * V;
#pragma unroll
      for (int i = 0; i < KPL; ++i) S[i] = (src && col_ok) ? src[e0 + i * V] : 0.f;
    }
  };

  // this lane's pieces of a block: piece p = lane + 64 j of each array
  uint4 rq[G::NQ], rk[G::NQ], rg[G::NG], rv[G::NV];
  auto issue = [&](const Unit &u, int64_t t0) __attribute__((always_inline)) {
    const int64_t rows = u.eos - t0;
    const int h = u.h;
    const char *qb = static_cast<const char *>(q) + t0 * H * G::QB;
    const char *kb = static_cast<const char *>(k) + t0 * H * G::QB;
    const char *gb = static_cast<const char *>(g) + t0 * H * G::GB;
    const char *vb = static_cast<const char *>(v) + t0 * H * static_cast<int64_t>(V) * G::ES;
    const auto rsq = rows_rsrc(qb, rows * H * G::QB), rsk = rows_rsrc(kb, rows * H * G::QB);
    const auto rsg = rows_rsrc(gb, rows * H * G::GB);
    const auto rsv = rows_rsrc(vb, rows * H * static_cast<int64_t>(V) * G::ES);
#pragma unroll
    for (int j = 0; j < G::NQ; ++j) {
      const int p = lane + 64 * j;
      const int st = p / (G::QB / 16), c = p % (G::QB / 16);
      const uint32_t off = p < G::PQ ? static_cast<uint32_t>((st * H + h) * G::QB + 16 * c) : kNoRow;
      rq[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsq, off, 0, 0));
      rk[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsk, off, 0, 0));
    }
#pragma unroll
    for (int j = 0; j < G::NG; ++j) {
      const int p = lane + 64 * j;
      const int st = p / (G::GB / 16), c = p % (G::GB / 16);
      const uint32_t off = p < G::PG ? static_cast<uint32_t>((st * H + h) * G::GB + 16 * c) : kNoRow;
      rg[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsg, off, 0, 0));
    }
#pragma unroll
    for (int j = 0; j < G::NV; ++j) {
      const int p = lane + 64 * j;
      const int st = p / (G::VB / 16), c = p % (G::VB / 16);
      const uint32_t off = p < G::PV ? static_cast<uint32_t>((static_cast<int64_t>(st) * H + h) * V * G::ES +
                                                             u.vt * G::VB + 16 * c)
                                     : kNoRow;
      rv[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsv, off, 0, 0));
    }
  };
  // q and k are parked as fp32: converted once per block element here, not
  // once per (step, lane) in the walk (the 16 lanes of a key group read the
  // same values)
  auto park_f32 = [&](unsigned char *dst, const uint4 &x) __attribute__((always_inline)) {
    if constexpr (DT == SSLA_F32) {
      *reinterpret_cast<uint4 *>(dst) = x;
    } else {
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
      float f[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint16_t b = static_cast<uint16_t>(w[c >> 1] >> (16 * (c & 1)));
        f[c] = DT == SSLA_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
      }
      *reinterpret_cast<float4 *>(dst) = make_float4(f[0], f[1], f[2], f[3]);
      *reinterpret_cast<float4 *>(dst + 16) = make_float4(f[4], f[5], f[6], f[7]);
    }
  };
  auto park = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < G::NQ; ++j) {
      const int p = lane + 64 * j;
      if (p < G::PQ) {   // piece p: row p / (QB / 16), elements 16 / ES * (p % (QB / 16)) ..
        const int off = (p / (G::QB / 16)) * G::DB + (p % (G::QB / 16)) * (16 / G::ES) * 4;
        park_f32(lds + G::OQ + off, rq[j]);
        park_f32(lds + G::OK + off, rk[j]);
      }
    }
    // decays of the block's gates: piece p holds 16 / GS gates, i.e.
    // 64 / GS bytes of fp32 decays at the same position of the decay rows
#pragma unroll
    for (int j = 0; j < G::NG; ++j) {
      const int p = lane + 64 * j;
      if (p < G::PG) {
        if constexpr (GDT == SSLA_F32) {
          const float4 x = __builtin_bit_cast(float4, rg[j]);
          *reinterpret_cast<float4 *>(lds + G::OD + 16 * p) =
              make_float4(fast_exp2(x.x * kLog2e), fast_exp2(x.y * kLog2e), fast_exp2(x.z * kLog2e),
                          fast_exp2(x.w * kLog2e));
        } else {
          const uint32_t w[4] = {rg[j].x, rg[j].y, rg[j].z, rg[j].w};
          float dd[8];
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const uint16_t b = static_cast<uint16_t>(w[c >> 1] >> (16 * (c & 1)));
            dd[c] = fast_exp2((GDT == SSLA_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b)) * kLog2e);
          }
          *reinterpret_cast<float4 *>(lds + G::OD + 32 * p) = make_float4(dd[0], dd[1], dd[2], dd[3]);
          *reinterpret_cast<float4 *>(lds + G::OD + 32 * p + 16) = make_float4(dd[4], dd[5], dd[6], dd[7]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < G::NV; ++j) {
      const int p = lane + 64 * j;
      if (p < G::PV) *reinterpret_cast<uint4 *>(lds + G::OV + 16 * p) = rv[j];
    }
  };

  const Unit cur = unit_at(static_cast<int>(blockIdx.x) * kRecWaves + wv);
  if (cur.bad && MODE != kSegState)
    skip_sequence<DT>(o, cur.bos, cur.eos, H, cur.h, V, col_of(cur), kg == 0 && col_of(cur) < V, lane, status);
  if (!cur.run) return;   // whole wavefront exits (no workgroup barrier)
  float S[KPL];
  init_state(cur, S);
  const int h = cur.h;
  const int col = col_of(cur);
  const bool col_ok = col < V;
  const int64_t e0 = elem0(cur);
  if (MODE == kSegOut) {
    // fold the earlier segments' local states, kFoldB per round trip (a
    // small batch: these registers count against the whole kernel's
    // allocation, and most sequences have few segments)
    for (int64_t j0 = 0; j0 < cur.seg; j0 += kFoldB) {
      float L[kFoldB][KPL], P[kFoldB][KPL];
#pragma unroll
      for (int u = 0; u < kFoldB; ++u) {
        const int64_t gj = cur.gseg - cur.seg + j0 + u;   // segment j0 + u of this sequence
        const bool ok = j0 + u < cur.seg;
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
          P[u][i] = ok ? sw.prod[(gj * H + h) * K + k0 + i] : 1.f;
          L[u][i] = (ok && col_ok) ? sw.slot[gj * H * K * V + e0 + i * V] : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < kFoldB; ++u)
#pragma unroll
        for (int i = 0; i < KPL; ++i) S[i] = fmaf(P[u][i], S[i], L[u][i]);
    }
  }
  float dprod[KPL];   // product of the decays of this unit (state pass)
#pragma unroll
  for (int i = 0; i < KPL; ++i) dprod[i] = 1.f;
  const int64_t nblk = (cur.eos - cur.bos + kSB - 1) / kSB;
  if (nblk > 0) issue(cur, cur.bos);
  for (int64_t b = 0; b < nblk; ++b) {
    const int64_t t0 = cur.bos + b * kSB;
    wave_lds_sync();   // the previous block's reads are done
    park();
    wave_lds_sync();
    if (b + 1 < nblk) issue(cur, t0 + kSB);
    const int ns = static_cast<int>(min(static_cast<int64_t>(kSB), cur.eos - t0));
    // o rows of this block's steps (step st of the block at (st H + h) V)
    const auto rso = rows_rsrc(static_cast<char *>(o) + (t0 * H + h) * static_cast<int64_t>(V) * G::ES,
                               ((ns - 1) * static_cast<int64_t>(H) + 1) * V * G::ES);
    // The steps of each half block (kHB steps) run without branches;
    // halves past the block's last step are skipped (a wavefront-uniform
    // branch).  Steps past the sequence end read the zero rows (decay 1,
    // k = q = 0: the state is unchanged) and store nothing.  The only
    // dependency carried from step to step is one fma per state
    // element.  Each step's partial dot product q . S over this lane's
    // keys stays in a register until the half is done; the sums over the
    // 4 key groups then run as lane swaps on the VALU, and key group kg
    // stores the steps s = kg mod 4 of the half.
    constexpr int kHB = kSB / 2;
    static_for<2>([&](auto hi) __attribute__((always_inline)) {
      constexpr int h0s = decltype(hi)::value * kHB;   // first step of this half
      if (h0s >= ns) return;
      float acc[kHB];
      static_for<kHB>([&](auto si) __attribute__((always_inline)) {
        constexpr int sl = decltype(si)::value;   // step within the half: acc index
        constexpr int st = h0s + sl;              // step within the block
        float d[KPL], kk[KPL], qs[KPL];
        if (MODE != kSegState) lds_run<SSLA_F32, KPL>(lds + G::OQ + st * G::DB + k0 * 4, qs);
        lds_run<SSLA_F32, KPL>(lds + G::OK + st * G::DB + k0 * 4, kk);
        lds_run<SSLA_F32, KPL>(lds + G::OD + st * G::DB + k0 * 4, d);
        const float vc = lds_elem<DT>(lds + G::OV + st * G::VB + (lane & 15) * G::ES);
        if (MODE == kSegState) {
#pragma unroll
          for (int i = 0; i < KPL; ++i) {
            S[i] = fmaf(d[i], S[i], kk[i] * vc);
            dprod[i] *= d[i];
          }
          return;
        }
        float a0 = 0.f, a1 = 0.f;   // two chains: half the dependent fma latency
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
          S[i] = fmaf(d[i], S[i], kk[i] * vc);
          if (i & 1) a1 = fmaf(qs[i], S[i], a1);
          else a0 = fmaf(qs[i], S[i], a0);
        }
        acc[sl] = a0 + a1;
        // computed here: otherwise the sums sink to the end of the half,
        // which keeps every step's updated state alive until then
        asm volatile("" : "+v"(acc[sl]));
      });
      if (MODE == kSegState) return;
      static_for<kHB / 4>([&](auto ji) __attribute__((always_inline)) {
        constexpr int j = decltype(ji)::value;
        const int st = h0s + 4 * j + kg;   // this key group's step; past ns: nothing stored
        const float x = sum4_key_groups(acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]);
        if (col_ok && st < ns)
          store_out<DT>(rso, static_cast<uint32_t>((st * H * V + col) * G::ES), x * scale);
      });
    });
  }
  if (MODE == kSegState) {
    if (col_ok) {
#pragma unroll
      for (int i = 0; i < KPL; ++i) sw.slot[static_cast<int64_t>(cur.gseg) * H * K * V + e0 + i * V] = S[i];
    }
    if (cur.vt == 0 && (lane & 15) == 0) {
#pragma unroll
      for (int i = 0; i < KPL; ++i) sw.prod[(static_cast<int64_t>(cur.gseg) * H + h) * K + k0 + i] = dprod[i];
    }
  } else if (ht && col_ok && cur.seg == cur.nseg - 1) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) ht[((static_cast<int64_t>(cur.srow) * H + h) * K + k0 + i) * V + col] = S[i];
  }
}

template <int DT, int GDT, int KPL>
__global__ __launch_bounds__(256) void gla_recurrent_kernel(
    const void *__restrict__ q, const void *__restrict__ k,
    const void *__restrict__ v, const void *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int H, int K, int V,
    float scale, const float *__restrict__ h0, void *__restrict__ o,
    float *__restrict__ ht, const int32_t *__restrict__ state_idx, int n_state_rows,
    int64_t T, int32_t *__restrict__ status) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int n_vt = (V + kBV - 1) / kBV;
  if (item >= static_cast<int64_t>(n_seq) * H * n_vt) return;  // whole wavefront exits
  const int vt = static_cast<int>(item % n_vt);
  const int h = static_cast<int>((item / n_vt) % H);
  const int n = static_cast<int>(item / (static_cast<int64_t>(n_vt) * H));

  const int col = vt * kBV + (lane & 15);   // value column of this lane
  const int kg = lane >> 4;                 // key group of this lane
  const int k0 = kg * KPL;                  // first key row of this lane
  const bool col_ok = col < V;

  // Clamp the sequence to [0, T) so that a malformed cu_seqlens can never
  // address memory outside q/k/v/g/o (the host wrapper reports it).
  const int64_t bos = min(max(cu_seqlens[n], (int64_t)0), T);
  const int64_t eos = min(max(cu_seqlens[n + 1], bos), T);
  const int64_t srow = state_idx ? static_cast<int64_t>(state_idx[n]) : n;
  if (bad_state_row(state_idx, n, srow, n_state_rows)) {   // never touch foreign rows
    skip_sequence<DT>(o, bos, eos, H, h, V, col, kg == 0 && col_ok, lane, status);
    return;
  }

  float S[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int kk = k0 + i;
    S[i] = (h0 && col_ok && kk < K) ? h0[((srow * H + h) * K + kk) * V + col] : 0.f;
  }

  typedef Elem<DT> E;
  typedef Elem<GDT> EG;
  for (int64_t t = bos; t < eos; ++t) {
    const int64_t qk_base = (t * H + h) * K;
    const float vv = col_ok ? E::load(v, (t * H + h) * V + col) : 0.f;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int kk = k0 + i;
      if (kk < K) {
        const float gg = EG::load(g, qk_base + kk);
        const float kv = E::load(k, qk_base + kk);
        const float qv = E::load(q, qk_base + kk);
        S[i] = fmaf(fast_exp2(gg * kLog2e), S[i], kv * vv);
        acc = fmaf(qv * scale, S[i], acc);
      }
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (kg == 0 && col_ok) E::store(o, (t * H + h) * V + col, acc);
  }

  if (ht && col_ok) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int kk = k0 + i;
      if (kk < K) ht[((srow * H + h) * K + kk) * V + col] = S[i];
    }
  }
}

// Workspace of the segmented schedule (0: not used for this shape -- K
// outside the staged kernels, or sequences of fewer than kSegAvgMin steps
// on average, where one pass is faster).
struct SegLayout {
  size_t segoff, segmap, slot, prod, h0c, total;
  int64_t n_segs_max;
  int seg_steps;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

inline SegLayout seg_layout(int n_seq, int64_t T, int H, int K, int V) {
  SegLayout L{};
  if (n_seq <= 0 || T <= 0 || K % 16 != 0 || K > 64 || V <= 0) return L;
  if (T < static_cast<int64_t>(n_seq) * kSegAvgMin) return L;
  // halve the segments (down to kSegStepsMin steps) while the grid holds
  // fewer than kSegUnits wavefronts -- shorter serial walks, more of them --
  // and sequences keep at most kSegFoldMax segments on average: segment s
  // folds the s local states before it, so the output pass grows with the
  // square of the segment count (at 20 per sequence it took longer than
  // the walks it saved)
  const int64_t n_vt = (V + kBV - 1) / kBV;
  L.seg_steps = kSegSteps;
  while (L.seg_steps > kSegStepsMin && (T / L.seg_steps + n_seq) * H * n_vt < kSegUnits &&
         T / (static_cast<int64_t>(n_seq) * (L.seg_steps / 2)) <= kSegFoldMax)
    L.seg_steps /= 2;
  L.n_segs_max = T / L.seg_steps + n_seq + 1;
  const size_t hkv = static_cast<size_t>(H) * K * V;
  size_t p = 0;
  L.segoff = p; p = align256(p + sizeof(int64_t) * (n_seq + 1));
  L.segmap = p; p = align256(p + sizeof(int4) * L.n_segs_max);
  L.slot = p;   p = align256(p + sizeof(float) * L.n_segs_max * hkv);
  L.prod = p;   p = align256(p + sizeof(float) * L.n_segs_max * H * K);
  L.h0c = p;    p = align256(p + sizeof(float) * n_seq * hkv);
  L.total = p;
  return L;
}

template <int DT, int GDT>
int launch_recurrent(const void *q, const void *k, const void *v, const void *g,
                     const int64_t *cu, int n_seq, int H, int K, int V, float scale,
                     const float *h0, void *o, float *ht, const int32_t *sidx,
                     int n_rows, int64_t T, int32_t *status, void *workspace, size_t ws_bytes,
                     hipStream_t st) {
  const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int n_vt = (V + kBV - 1) / kBV;
  const int64_t items = static_cast<int64_t>(n_seq) * H * n_vt;
  if (items == 0) return SSLA_OK;
  const int waves_per_block = kRecWaves;
  const int64_t blocks = (items + waves_per_block - 1) / waves_per_block;
  if (blocks > 0x7fffffff) {
    set_error("gla_recurrent_fwd: too many (sequence, head, tile) items");
    return SSLA_ERR_UNSUPPORTED;
  }
  dim3 grid(static_cast<unsigned>(blocks)), block(64 * waves_per_block);
  const int kpl_needed = (K + kKG - 1) / kKG;
  // staged path: every lane's run of keys is whole (K = 4 KPL <= 64), and
  // q/k/g rows and the v rows are whole 16-byte pieces at 16-byte aligned
  // addresses
  const int es = DT == SSLA_F32 ? 4 : 2;
  const bool staged = (K % 16 == 0) && K <= 64 && (V * es) % 16 == 0 && al16(q) && al16(k) && al16(g) && al16(v);
  if (staged) {
    // one wavefront per unit; unit indices are 32-bit in the kernel
    const SegLayout L = seg_layout(n_seq, T, H, K, V);
    const bool segmented = L.total > 0 && workspace != nullptr && ws_bytes >= L.total;
    if (items > 0x7fffffff || (segmented && L.n_segs_max * H * n_vt > 0x7fffffff)) {
      set_error("gla_recurrent_fwd: too many (sequence or segment, head, tile) items");
      return SSLA_ERR_UNSUPPORTED;
    }
    SegWs sw{};
    dim3 sgrid = grid;
    if (segmented) {
      char *w = static_cast<char *>(workspace);
      sw.segoff = reinterpret_cast<const int64_t *>(w + L.segoff);
      sw.segmap = reinterpret_cast<const int4 *>(w + L.segmap);
      sw.slot = reinterpret_cast<float *>(w + L.slot);
      sw.prod = reinterpret_cast<float *>(w + L.prod);
      sw.h0c = reinterpret_cast<float *>(w + L.h0c);
      sw.n_segs_max = L.n_segs_max;
      sw.seg_steps = L.seg_steps;
      sgrid = dim3(static_cast<unsigned>((L.n_segs_max * H * n_vt + waves_per_block - 1) / waves_per_block));
      hipLaunchKernelGGL(seg_offsets_kernel, dim3(1), dim3(256), 0, st, cu, n_seq, T, L.seg_steps, L.n_segs_max,
                         reinterpret_cast<int64_t *>(w + L.segoff), reinterpret_cast<int4 *>(w + L.segmap),
                         status);
    }
#define SSLA_RECS(KPL_)                                                                                     \
  if (segmented) {                                                                                          \
    hipLaunchKernelGGL((gla_recurrent_staged_kernel<DT, GDT, KPL_, kSegState>), sgrid, block, 0, st, q, k, v, \
                       g, cu, n_seq, H, V, scale, h0, o, ht, sidx, n_rows, T, status, sw);                  \
    hipLaunchKernelGGL((gla_recurrent_staged_kernel<DT, GDT, KPL_, kSegOut>), sgrid, block, 0, st, q, k, v,   \
                       g, cu, n_seq, H, V, scale, h0, o, ht, sidx, n_rows, T, status, sw);                  \
  } else {                                                                                                  \
    hipLaunchKernelGGL((gla_recurrent_staged_kernel<DT, GDT, KPL_, kPlain>), grid, block, 0, st, q, k, v, g,  \
                       cu, n_seq, H, V, scale, h0, o, ht, sidx, n_rows, T, status, sw);                     \
  }
    switch (K / kKG) {
      case 4: SSLA_RECS(4); return launch_status("gla_recurrent_fwd");
      case 8: SSLA_RECS(8); return launch_status("gla_recurrent_fwd");
      case 16: SSLA_RECS(16); return launch_status("gla_recurrent_fwd");
      default: break;   // other K: the general kernel
    }
#undef SSLA_RECS
  }
#define SSLA_REC(KPL_)                                                                     \
  hipLaunchKernelGGL((gla_recurrent_kernel<DT, GDT, KPL_>), grid, block, 0, st, q, k, v, g, \
                     cu, n_seq, H, K, V, scale, h0, o, ht, sidx, n_rows, T, status)
  if (kpl_needed <= 4) SSLA_REC(4);
  else if (kpl_needed <= 8) SSLA_REC(8);
  else if (kpl_needed <= 16) SSLA_REC(16);
  else if (kpl_needed <= 32) SSLA_REC(32);
  else SSLA_REC(64);
#undef SSLA_REC
  return launch_status("gla_recurrent_fwd");
}

}  // namespace
}  // namespace ssla

extern "C" int ssla_gla_recurrent_fwd(const void *q, const void *k, const void *v,
                                      const void *g, int g_dtype,
                                      const int64_t *cu_seqlens, int n_seq, int64_t T,
                                      int H, int K, int V, float scale,
                                      const float *h0, void *o, float *ht,
                                      const int32_t *state_idx, int n_state_rows,
                                      int32_t *status, int dtype, void *workspace,
                                      size_t workspace_bytes, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && T >= 0 && H > 0 && K > 0 && V > 0,
                 "gla_recurrent_fwd: bad sizes n_seq=%d T=%lld H=%d K=%d V=%d", n_seq,
                 (long long)T, H, K, V);
  if (K > 256 || V > 256) {
    set_error("gla_recurrent_fwd: K=%d V=%d exceed 256", K, V);
    return SSLA_ERR_UNSUPPORTED;
  }
  if (n_seq == 0) return SSLA_OK;
  SSLA_CHECK_ARG(cu_seqlens != nullptr, "gla_recurrent_fwd: cu_seqlens is NULL");
  SSLA_CHECK_ARG(T == 0 || (q && k && v && g && o), "gla_recurrent_fwd: null tensor pointer");
  SSLA_CHECK_ARG(state_idx == nullptr || n_state_rows > 0,
                 "gla_recurrent_fwd: state_idx given with n_state_rows=%d", n_state_rows);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SSLA_F32) {
    if (g_dtype != SSLA_F32) { set_error("gla_recurrent_fwd: fp32 inputs need fp32 g"); return SSLA_ERR_DTYPE; }
    return launch_recurrent<SSLA_F32, SSLA_F32>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, workspace, workspace_bytes, st);
  }
  if (dtype == SSLA_BF16) {
    if (g_dtype == SSLA_F32)
      return launch_recurrent<SSLA_BF16, SSLA_F32>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, workspace, workspace_bytes, st);
    if (g_dtype == SSLA_BF16)
      return launch_recurrent<SSLA_BF16, SSLA_BF16>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, workspace, workspace_bytes, st);
  }
  if (dtype == SSLA_F16) {
    if (g_dtype == SSLA_F32)
      return launch_recurrent<SSLA_F16, SSLA_F32>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, workspace, workspace_bytes, st);
    if (g_dtype == SSLA_F16)
      return launch_recurrent<SSLA_F16, SSLA_F16>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, workspace, workspace_bytes, st);
  }
  set_error("gla_recurrent_fwd: unsupported dtype %d / g_dtype %d", dtype, g_dtype);
  return SSLA_ERR_DTYPE;
}

extern "C" size_t ssla_gla_recurrent_workspace_size(int n_seq, int64_t T, int H, int K, int V) {
  if (H <= 0) return 0;
  return ssla::seg_layout(n_seq, T, H, K, V).total;
}
