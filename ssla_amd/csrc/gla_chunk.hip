// Chunked gated-linear-attention forward on gfx950.
//
// Math (reference ops/gla/chunk.py:906-960 with ops/utils/cumsum.py:61-90,
// ops/common/chunk_h.py:27-128 and ops/gla/chunk.py:33-249): per sequence
// and head, split time into chunks of 64 rows (chunks restart at every
// sequence start) and with G the chunk-local inclusive cumsum of the
// log-gates g:
//   o_c   = (scale q_c * exp(G)) S_c + tril(A_c) v_c,
//   A_ij  = scale sum_k q_ik k_jk exp(G_ik - G_jk)                 (j <= i)
//   S_c+1 = diag(exp(G_last)) S_c + (k_c * exp(G_last - G))^T v_c
// with S_0 = h0 (or 0) and ht = S after the last chunk.
//
// Schedule (two launches; the only intermediates are per-segment states):
// * Each (sequence, head, V group) chain is cut into P segments of whole
//   chunks (P chosen so that about two workgroups run per CU).
// * state pass  : segments 0..P-2 run the state recurrence only (reads k, g,
//   v) from h0 (segment 0) or zero, leaving the segment's final state and
//   total log2-decay D in a workspace slot.  The state is stored as a bf16
//   pair: hi = bf16(S) and lo = bf16(S - hi), so hi + lo holds S to about
//   2^-17.
// * segment pass: every segment first folds the slots of the segments before
//   it into its entering state (E = slot 0, E = 2^D(j) E + slot j for
//   0 < j < s), then runs the full chunk loop from it and writes o (and ht
//   for the last segment).  The fold uses the hi halves: the entering state
//   reaches o through a product in the input dtype, as the reference's
//   per-chunk states do (bf16 at states_in_fp32=False).  The last segment,
//   whose final state becomes ht, adds the fold of the lo halves at the end,
//   decayed through its own chunks (the fold is linear, so
//   ht = S(fold(hi)) + decay * fold(lo)): ht carries fp32-level accuracy
//   across segments without delaying the segment's first chunk.
//
// Inside a workgroup (256 threads, 4 wavefronts): wavefront I owns chunk
// rows 16I..16I+15 ("block" I) and state rows (keys) 16I..16I+15 as MFMA
// accumulators.  All products are v_mfma_f32_16x16x32_{bf16,f16}.  Within a
// lane the 64 keys are held as k = 32*jj + 8*(lane/16) + e (jj = 0,1; e =
// 0..7), the operand layout of the two K=32 halves of a K=64 product.
// Products that contract over time (A v, k^T v) read their operands from
// row-major LDS tiles with ds_read_b64_tr_b16 (transposing 16-bit loads),
// so no transposed copies are written.
//
// Decay factorisation (log2 units, G2 = G * log2(e)), per key and block I
// with block boundary values E_J (G2 at the last row of block J, E_-1 = 0)
// and M_I = (E_I-1 + E_I) / 2:
//   diagonal block     : 2^(G_i - G_j) = 2^(G_i - M_I) 2^(M_I - G_j)
//   block J < I        : 2^(G_i - G_j) = [2^(G_i - M_I) 2^(M_I - E_J)] [2^(E_J - G_j)]
// For non-positive gates the off-diagonal factors are all <= 1 (exact up to
// underflow of values that are themselves below 2^-126), and the diagonal
// factors stay inside 2^(+-x) with x the decay over half a block (8 rows);
// exponents are clamped to +-126, which only matters when a key decays by
// more than 2^-126 within 8 steps.  The state enters the output product in
// the input dtype, as the reference's per-chunk states do
// (states_in_fp32=False, ops/gla/chunk.py:933).  scale is applied to o at
// the end.
#include "lds_tile.h"

#include <atomic>
#include <mutex>
#include <type_traits>

// Scratch of ssla_gla_chunk_fwd_noalloc: a fixed device array (one copy per
// GPU, zero-filled when the code object loads, held until the process
// ends) that stands in for the caller's workspace.  Host code never passes
// its name to a kernel: the name is a host-side stand-in; the device address
// comes from hipGetSymbolAddress (noalloc_scratch below).
static constexpr size_t kNoallocScratchBytes = size_t{64} << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace ssla {
namespace {

constexpr int BT = 64;    // chunk rows
constexpr int KD = 64;    // key width
constexpr float kExpClamp = 126.f;
#ifndef SSLA_GC_STATE_WAVES
#define SSLA_GC_STATE_WAVES 3
#endif
#ifndef SSLA_GC_SEG_WAVES
#define SSLA_GC_SEG_WAVES 2
#endif

typedef float f32x8 __attribute__((ext_vector_type(8)));

// MFMA of the input dtype (value products: S^T q0, V^T A^T, k^T v).
template <int DT> struct Mfma;
template <> struct Mfma<SSLA_BF16> {
  typedef bf16x8 Vec;
  static __device__ __forceinline__ f32x4 mma(Vec a, Vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ Vec cvt(f32x8 x) { return __builtin_convertvector(x, bf16x8); }
  static __device__ __forceinline__ f32x8 widen(Vec x) { return __builtin_convertvector(x, f32x8); }
};
template <> struct Mfma<SSLA_F16> {
  typedef f16x8 Vec;
  static __device__ __forceinline__ f32x4 mma(Vec a, Vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ Vec cvt(f32x8 x) { return __builtin_convertvector(x, f16x8); }
  static __device__ __forceinline__ f32x8 widen(Vec x) { return __builtin_convertvector(x, f32x8); }
};
// The decayed q~ k~^T products always run in bf16: its fp32 exponent range
// holds factors that fp16 cannot.
typedef Mfma<SSLA_BF16> QK;

// Row staging of one wavefront (its 16 chunk rows), byte layout:
// * q, k (and 16-bit g): pieces 0-3 and 4-7 of a row (16 bytes each) in
//   two half tiles kHalf bytes apart; row r at 64 r (+32 for r >= 8), piece
//   p at slot (p & 3) ^ s(r) with s(r) = (r >> 2) & 1;
// * fp32 g: pieces 4q'..4q'+3 in quarter tile q' (kQuart bytes apart); row r
//   at 64 r (+16 for r >= 8), piece p at slot (p & 3) ^ 2 s(r).
// Every access of a lane is then one base address plus immediate offsets,
// and both the whole-line writes and the MFMA-layout reads (16 rows, one
// piece each) spread over the 64 banks (at most two lanes of a 16-lane
// group per bank).
constexpr int kHalf = 1152, kQuart = 1152;
constexpr int kTileQK = 2 * kHalf, kTileG = 4 * kQuart;
template <bool Q> struct RowStage;
template <> struct __align__(16) RowStage<true> { unsigned char q[kTileQK], k[kTileQK], g[kTileG]; };
template <> struct __align__(16) RowStage<false> { unsigned char k[kTileQK], g[kTileG]; };

__device__ __forceinline__ int stage_qk_off(int r, int p) {
  return (p >> 2) * kHalf + 64 * r + (r >= 8 ? 32 : 0) + 16 * ((p & 3) ^ ((r >> 2) & 1));
}
__device__ __forceinline__ int stage_g_off(int r, int p) {
  return (p >> 2) * kQuart + 64 * r + (r >= 8 ? 16 : 0) + 16 * ((p & 3) ^ (2 * ((r >> 2) & 1)));
}

struct __align__(16) SmemA {
  uint16_t sth[64 * 64];   // S^T (column v, key k), input dtype
  uint16_t kt[64 * 64];    // k 2^(E_J - G) rows (bf16), blocks read by later wavefronts
  uint16_t kh[64 * 64];    // k 2^(G_last - G) rows (input dtype)
  uint16_t vs[64 * 64];    // v rows of the V group (input dtype)
  float tot[4][KD];        // per-block column sums of g (log2 units)
  float fac[4][8][KD];     // per-wavefront per-key factors (slots below)
};
constexpr int kFacHalf = 0;  // M_I - E_I-1          (G2 - it = G_abs - M_I)
constexpr int kFacQ0 = 1;    // 2^M_I                (q0 = q~ 2^M_I)
constexpr int kFacKh = 2;    // 2^(G_last - M_I)     (k^ = k~ 2^(G_last - M_I))
constexpr int kFacKt = 3;    // 2^(E_I - M_I)        (kt = k~ 2^(E_I - M_I))
constexpr int kFacDec = 4;   // 2^G_last             (state decay)
constexpr int kFacQJ = 5;    // 2^(M_I - E_J), J < I (q~ for block J)

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier that orders LDS only: prefetched global loads stay in
// flight across it (a full __syncthreads() would drain them every chunk).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 16 independent inclusive row scans, step-major so that consecutive DPP
// instructions never depend on each other.
template <int N>
__device__ __forceinline__ void row_scan_step(f32x8 (&x)[2]) {
  f32x8 t[2];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
#pragma unroll
    for (int e = 0; e < 8; ++e) t[jj][e] = row_shr<N>(x[jj][e]);
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) x[jj] += t[jj];
}
__device__ __forceinline__ void row_scan16(f32x8 (&x)[2]) {
  row_scan_step<1>(x);
  row_scan_step<2>(x);
  row_scan_step<4>(x);
  row_scan_step<8>(x);
}

__device__ __forceinline__ float clamp_exp(float x) { return fminf(fmaxf(x, -kExpClamp), kExpClamp); }

// One chunk row of this lane in the MFMA operand layout: q, k, g at keys
// {kq..kq+7, 32+kq..32+kq+7} of row r (filled from the row staging).
struct ChunkRegs {
  uint4 q[2], k[2];   // 16-bit
  float4 g[4];        // fp32 g ...
  uint4 g16[2];       // ... or 16-bit g
};

// The segment kernel loads straight into the MFMA layout (its registers
// leave no room for the staging copy): ChunkRegs plus this lane's v pieces.
struct SegRegs : ChunkRegs {
  uint4 v[2];
};

// Whole-line loads of one chunk: wavefront w reads its rows 16w..16w+15,
// eight lanes per 128-byte row of q / k / v / 16-bit g (row 16w + 8i +
// lane/8, 16-byte piece lane%8 in instruction i) and sixteen lanes per
// 256-byte row of fp32 g (row 16w + 4i + lane/16, piece lane%16).  Whole
// lines per instruction stream about 1.35x faster from HBM than the MFMA
// layout's half lines; q, k, g are then transposed through LDS
// (stage_rows) and v goes to its tile as it is.
struct LineRegs {
  uint4 q[2], k[2], v[2], g[4];
};


// Per-sequence buffer resources of q, k, g, v and o: the base is the
// sequence's first row and the size its rows, so the hardware range check
// returns zeros for loads of rows past the sequence end and drops stores to
// them.  Rows past the end therefore need no branches: zero g keeps the
// chunk's total decay at the last valid row, zero k / v remove them from the
// state update, and their outputs are never written.  Offsets are 32-bit
// byte offsets (the host checks that a sequence stays below 2 GB).
struct SeqRsrc {
  __amdgpu_buffer_rsrc_t q, k, g, v, o;
};

constexpr int kRsrcWord3 = 0x00020000;   // raw 32-bit data, range checked
constexpr uint32_t kNoLoad = 0x80000000u; // an offset past every resource: reads zeros, no traffic

__device__ __forceinline__ __amdgpu_buffer_rsrc_t seq_rsrc(const void *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), kRsrcWord3);
}

// Byte offsets (inside the sequence resources) of this lane's first
// whole-line load of a chunk, and the steps between its instructions.
struct LineOffs {
  uint32_t a16;   // q / k (and 16-bit g): row 16w + lane/8, piece lane%8
  uint32_t g;     // fp32 g: row 16w + lane/16, piece lane%16
  uint32_t v;     // v: row 16w + lane/8, columns v0 + 8 (lane%8)
};

__device__ __forceinline__ LineOffs line_offs(int c, int wv, int lane, int H, int h, int V, int v0, int gsz) {
  LineOffs o;
  const uint32_t r8 = static_cast<uint32_t>((c * BT + 16 * wv + (lane >> 3)) * H + h);
  const uint32_t r16 = static_cast<uint32_t>((c * BT + 16 * wv + (lane >> 4)) * H + h);
  o.a16 = r8 * (KD * 2) + 16 * (lane & 7);
  o.g = gsz == 4 ? r16 * (KD * 4) + 16 * (lane & 15) : o.a16;
  o.v = r8 * static_cast<uint32_t>(V * 2) + static_cast<uint32_t>(v0 * 2) + 16 * (lane & 7);
  return o;
}

// Issue the whole-line loads of one chunk.  `valid` false (no next chunk)
// turns every load into a zero read without memory traffic, so the
// instruction stream is the same on every iteration; v pieces beyond the V
// group (vcol_ok false) read zeros as well.
template <bool LOADQ, bool GF32>
__device__ __forceinline__ void load_lines(LineRegs &L, const SeqRsrc &rs, bool valid, const LineOffs &o, int H,
                                           int V, bool vcol_ok) {
  const uint32_t a = valid ? o.a16 : kNoLoad, b = valid ? o.g : kNoLoad, c = (valid && vcol_ok) ? o.v : kNoLoad;
  const uint32_t s16 = 8 * H * KD * 2, sg = 4 * H * KD * 4, sv = 8 * H * V * 2;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (LOADQ) L.q[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.q, a + i * s16, 0, 0));
    L.k[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.k, a + i * s16, 0, 0));
    L.v[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.v, c + i * sv, 0, 0));
  }
  if (GF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      L.g[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.g, b + i * sg, 0, 0));
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      L.g[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.g, b + i * s16, 0, 0));
  }
}

// Write the chunk's lines into the wavefront's staging and read them back
// in the MFMA layout (lane 16 gq + r: row r, pieces gq and 4 + gq; fp32 g
// pieces 8 jj + 2 gq + {0, 1}).  The staging is private to the wavefront.
template <bool LOADQ, bool GF32>
__device__ __forceinline__ void stage_rows(RowStage<LOADQ> &st, const LineRegs &L, int lane, ChunkRegs &R) {
  const int r = lane & 15, gq = lane >> 4;
  auto at = [](unsigned char *base, int off) __attribute__((always_inline)) {
    return reinterpret_cast<uint4 *>(base + off);
  };
  // whole-line writes: 16-bit rows lane/8 (+8), fp32 g rows lane/16 + 4i
  const int w16 = stage_qk_off(lane >> 3, lane & 7);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if constexpr (LOADQ) *at(st.q, w16 + 544 * i) = L.q[i];
    *at(st.k, w16 + 544 * i) = L.k[i];
    if (!GF32) *at(st.g, w16 + 544 * i) = L.g[i];
  }
  if (GF32) {
    const int wg0 = stage_g_off(lane >> 4, lane & 15), wg1 = stage_g_off(4 + (lane >> 4), lane & 15);
    *at(st.g, wg0) = L.g[0];
    *at(st.g, wg1) = L.g[1];
    *at(st.g, wg0 + 528) = L.g[2];
    *at(st.g, wg1 + 528) = L.g[3];
  }
  wave_sync_lds();
  const int r16 = stage_qk_off(r, gq);
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    if constexpr (LOADQ) R.q[jj] = *at(st.q, r16 + kHalf * jj);
    R.k[jj] = *at(st.k, r16 + kHalf * jj);
    if (!GF32) R.g16[jj] = *at(st.g, r16 + kHalf * jj);
  }
  if (GF32) {
    const int rg = stage_g_off(r, 2 * gq);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        R.g[2 * jj + h2] = __builtin_bit_cast(float4, *at(st.g, rg + 2 * kQuart * jj + 16 * h2));
  }
}

// v lines of this wavefront's rows into the V tile (columns beyond the V
// group are skipped).
__device__ __forceinline__ void store_v_lines(uint16_t *vs, const LineRegs &L, int wv, int lane, int vw) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 16 * wv + 8 * i + (lane >> 3), col = 8 * (lane & 7);
    if (col < vw) tile_store8(vs, row, col, L.v[i]);
  }
}

// Raw loads of one chunk row of this lane: q, k, g at keys {kq..kq+7,
// 32+kq..32+kq+7} and v at columns {kq.., 32+kq..} of its V group.  oq / og /
// ov are the byte offsets of the lane's first element; `valid` false (no
// next chunk) turns every load into a zero read without memory traffic, so
// the instruction stream is the same on every iteration.
template <bool LOADQ, bool GF32>
__device__ __forceinline__ void load_chunk(SegRegs &R, const SeqRsrc &rs, bool valid, uint32_t oq,
                                           uint32_t og, uint32_t ov, int kq, int vw) {
  const uint32_t q0 = valid ? oq : kNoLoad, g0 = valid ? og : kNoLoad;
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    if (LOADQ) R.q[jj] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.q, q0 + 64 * jj, 0, 0));
    R.k[jj] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.k, q0 + 64 * jj, 0, 0));
    if (GF32) {
      R.g[2 * jj] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs.g, g0 + 128 * jj, 0, 0));
      R.g[2 * jj + 1] =
          __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs.g, g0 + 128 * jj + 16, 0, 0));
    } else {
      R.g16[jj] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.g, g0 + 64 * jj, 0, 0));
    }
    // columns beyond the V group are never used: read zeros instead
    const uint32_t vo = (valid && 32 * jj + kq < vw) ? ov + 64 * jj : kNoLoad;
    R.v[jj] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.v, vo, 0, 0));
  }
}

// Unpack 16 gates (log2 units) of this lane.
template <int DT, bool GF32>
__device__ __forceinline__ void unpack_gates(const ChunkRegs &R, f32x8 (&gs)[2]) {
  typedef Mfma<DT> M;
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    if (GF32) {
      const f32x4 x0 = __builtin_bit_cast(f32x4, R.g[2 * jj]), x1 = __builtin_bit_cast(f32x4, R.g[2 * jj + 1]);
      gs[jj] = (f32x8){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]} * kLog2e;
    } else {
      gs[jj] = M::widen(from_bits<typename M::Vec>(R.g16[jj])) * kLog2e;
    }
  }
}

// S (fp32 accumulator tile: keys krow..krow+3, column vcol) -> S^T tile in
// the input dtype.
template <int DT>
__device__ __forceinline__ void store_state(uint16_t *sth, int vcol, int krow, const f32x4 &S) {
  typedef Mfma<DT> M;
  const f32x8 s8 = {S[0], S[1], S[2], S[3], 0.f, 0.f, 0.f, 0.f};
  const uint4 b = to_bits(M::cvt(s8));
  *reinterpret_cast<uint2 *>(sth + swz(vcol, krow)) = make_uint2(b.x, b.y);
}

// Position of a lane's accumulator tiles inside a workspace slot: the
// state pass writes, and the segment pass reads, the 4*NVT values of each
// lane (tile t, rows i) as one contiguous run, so both use 8-byte accesses.
template <int NVT>
__device__ __forceinline__ int64_t slot_index(int v0, int wv, int lane) {
  return static_cast<int64_t>((v0 / (16 * NVT) * 4 + wv) * 64 + lane) * (4 * NVT);
}

// Four bf16 values (packed low half first) -> fp32.
__device__ __forceinline__ void unpack_bf16x4(const uint2 &b, float (&x)[4]) {
  x[0] = __uint_as_float(b.x << 16);
  x[1] = __uint_as_float(b.x & 0xffff0000u);
  x[2] = __uint_as_float(b.y << 16);
  x[3] = __uint_as_float(b.y & 0xffff0000u);
}

struct ChunkArgs {
  const uint16_t *q, *k, *v;
  const void *g;
  const float *h0;
  uint16_t *o;
  float *ht;
  const uint16_t *ws_state;  // [n_seq, H, P] slots of K*V bf16 in slot_index order: local end state of segment s (hi)
  const uint16_t *ws_lo;     // the same slots: bf16(S - hi)
  const float *ws_decay;   // [n_seq, H, P, K] fp32: total log2 decay of segment s
  int64_t bos;             // first row of the sequence
  int64_t len;             // rows of the sequence
  int c_beg, c_end;        // chunk range of the segment
  int H, V, h, n, v0, seg, P;
  float scale;
};

// Chunk range of segment `seg` of a sequence with `nch` chunks cut in P parts.
__device__ __forceinline__ void segment_range(int nch, int P, int seg, int &c0, int &c1) {
  const int per = (nch + P - 1) / P;
  c0 = min(seg * per, nch);
  c1 = min(c0 + per, nch);
}

// E = slot 0, E = 2^D(j) E + slot j for 0 < j < a.seg (in this order, so
// every segment gets the same bits), over this lane's values of the hi
// halves (LO = false) or the lo halves (LO = true).  Slots and decays are
// loaded eight at a time, so up to 8 segments take one round trip.
template <int NVT, bool LO>
__device__ __forceinline__ void fold_slots(const struct ChunkArgs &a, int64_t sl0, const float *dk, f32x4 (&S)[NVT]) {
  const uint16_t *base = LO ? a.ws_lo : a.ws_state;
  for (int j0 = 0; j0 < a.seg; j0 += 8) {
    uint2 xb[8][NVT];
    f32x4 d[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (j0 + u < a.seg) {
        const int64_t so = sl0 + static_cast<int64_t>(j0 + u) * KD * a.V;
        d[u] = *reinterpret_cast<const f32x4 *>(dk + static_cast<int64_t>(j0 + u) * KD);
#pragma unroll
        for (int t = 0; t < NVT; ++t) xb[u][t] = *reinterpret_cast<const uint2 *>(base + so + 4 * t);
      }
    }
    float x[8][NVT][4];
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int t = 0; t < NVT; ++t) unpack_bf16x4(xb[u][t], x[u][t]);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u;
      if (j == 0) {
#pragma unroll
        for (int t = 0; t < NVT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) S[t][i] = x[u][t][i];
      } else if (j < a.seg) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float f = fast_exp2(clamp_exp(d[u][i]));
#pragma unroll
          for (int t = 0; t < NVT; ++t) S[t][i] = fmaf(f, S[t][i], x[u][t][i]);
        }
      }
    }
  }
}

// --------------------------------------------------------- segment pass --
template <int DT, bool GF32, int NVT>
__device__ __forceinline__ void segment_loop(SmemA &sm, const ChunkArgs &a, const int wv, int lane) {
  typedef Mfma<DT> M;
  typedef typename M::Vec MV;
  const int r = lane & 15;        // row within block / MFMA column index
  const int gq = lane >> 4;       // lane group
  const int kq = 8 * gq;          // key offset of this lane inside each K=32 half
  const int H = a.H, V = a.V, h = a.h, v0 = a.v0;
  const int vw = 16 * NVT;        // columns of the V group
  const int64_t len = a.len;

  // ---- entering state: keys 16wv + 4gq + i, columns v0 + 16t + r ---------
  const int64_t sbase = (static_cast<int64_t>(a.n) * H + h) * KD;
  const int krow = 16 * wv + 4 * gq;
  // the first chunk's loads go out before the entering state is read
  const int row = 16 * wv + r;
  constexpr int gsz = GF32 ? 4 : 2;   // bytes per g element
  SeqRsrc rs;
  rs.q = seq_rsrc(a.q + a.bos * H * KD, len * H * KD * 2);
  rs.k = seq_rsrc(a.k + a.bos * H * KD, len * H * KD * 2);
  rs.g = seq_rsrc(static_cast<const char *>(a.g) + a.bos * H * KD * gsz, len * H * KD * gsz);
  rs.v = seq_rsrc(a.v + a.bos * H * V, len * H * V * 2);
  rs.o = seq_rsrc(a.o + a.bos * H * V, len * H * V * 2);
  // byte offsets of this lane's row (chunk c_beg) inside the sequence, and
  // their per-chunk steps
  const uint32_t rowi = static_cast<uint32_t>((a.c_beg * BT + row) * H + h);
  uint32_t oq = (rowi * KD + kq) * 2, og = (rowi * KD + kq) * gsz;
  uint32_t ov = (rowi * V + v0) * 2;   // row start of the V group (o uses it too)
  const uint32_t sq = BT * H * KD * 2, sg = BT * H * KD * gsz, sv = BT * H * V * 2;
  SegRegs buf;
  load_chunk<true, GF32>(buf, rs, a.c_beg < a.c_end, oq, og, ov + 2 * kq, kq, vw);
  f32x4 S[NVT];
  {
    // entering state: h0 for segment 0, else the fold of the earlier
    // segments' slots, E = slot 0, E = 2^D(j) E + slot j for 0 < j < seg (in
    // this order, so every segment gets the same bits); slots and decays are
    // loaded in batches (8, or 4 with the lo halves), so up to 8 segments
    // take one or two round trips
    const int64_t chain = static_cast<int64_t>(a.n) * H + h;
    const int64_t eo = static_cast<int64_t>(krow) * V + v0 + r;   // this lane's element (i = 0, t = 0)
    if (a.seg == 0) {
      const float *src = a.h0 ? a.h0 + sbase * V : nullptr;
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[t][i] = src ? src[eo + static_cast<int64_t>(i) * V + 16 * t] : 0.f;
    } else {
      const int64_t sl0 = chain * a.P * KD * V + slot_index<NVT>(a.v0, wv, lane);
      const float *dk = a.ws_decay + chain * a.P * KD + krow;
      fold_slots<NVT, false>(a, sl0, dk, S);
    }
  }
  // Wait here for the entering state (and the first chunk, needed next
  // anyway): otherwise the loop's wait bookkeeping carries these loads
  // around the back edge and drains all loads (vmcnt(0)) in every chunk.
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0) only


  // Two prefetch register sets used in turn (the loop is unrolled by two),
  // so no copy is made and the wait at each chunk covers only the loads of
  // that chunk, not the o stores issued after them.
  SegRegs buf2;
  f32x4 dec_prod = {1.f, 1.f, 1.f, 1.f};   // decay of this lane's state rows over the segment
  auto chunk_step = [&](SegRegs &cur, SegRegs &nxt, const int c) __attribute__((always_inline)) {
    const uint32_t orow = ov;   // o row of this lane in this chunk (same layout as v)

    // ---- prefetch q, k, g, v of c+1 -------------------------------------------
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    oq += sq;
    og += sg;
    ov += sv;
    load_chunk<true, GF32>(nxt, rs, c + 1 < a.c_end, oq, og, ov + 2 * kq, kq, vw);
    __builtin_amdgcn_sched_barrier(0);

    // ---- block-local inclusive cumsum over the 16 rows (DPP row scan) ------
    f32x8 gs[2];
    unpack_gates<DT, GF32>(cur, gs);
    row_scan16(gs);
    if (r == 15) {
      *reinterpret_cast<f32x8 *>(&sm.tot[wv][kq]) = gs[0];
      *reinterpret_cast<f32x8 *>(&sm.tot[wv][32 + kq]) = gs[1];
    }
    lds_barrier();  // --------------------------------------------- barrier 1
    // Every wavefront finished chunk c-1, so sth / kt / kh / vs are free.

    // ---- per-key factors (lane = key) --------------------------------------
    {
      const int kk = lane;
      const float E0 = sm.tot[0][kk];
      const float E1 = E0 + sm.tot[1][kk];
      const float E2 = E1 + sm.tot[2][kk];
      const float E3 = E2 + sm.tot[3][kk];
      const float Ep = wv == 0 ? 0.f : wv == 1 ? E0 : wv == 2 ? E1 : E2;
      const float Eo = wv == 0 ? E0 : wv == 1 ? E1 : wv == 2 ? E2 : E3;
      const float Mi = 0.5f * (Ep + Eo);
      sm.fac[wv][kFacHalf][kk] = Mi - Ep;
      sm.fac[wv][kFacQ0][kk] = fast_exp2(clamp_exp(Mi));
      sm.fac[wv][kFacKh][kk] = fast_exp2(clamp_exp(E3 - Mi));
      sm.fac[wv][kFacKt][kk] = fast_exp2(clamp_exp(Eo - Mi));
      sm.fac[wv][kFacDec][kk] = fast_exp2(clamp_exp(E3));
      if (wv > 0) sm.fac[wv][kFacQJ + 0][kk] = fast_exp2(clamp_exp(Mi - E0));
      if (wv > 1) sm.fac[wv][kFacQJ + 1][kk] = fast_exp2(clamp_exp(Mi - E1));
      if (wv > 2) sm.fac[wv][kFacQJ + 2][kk] = fast_exp2(clamp_exp(Mi - E2));
    }
    // the state entering this chunk (S^T in the input dtype) and the V rows
#pragma unroll
    for (int t = 0; t < NVT; ++t) store_state<DT>(sm.sth, 16 * t + r, krow, S[t]);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
      if (32 * jj + kq < vw) tile_store8(sm.vs, row, 32 * jj + kq, cur.v[jj]);
    wave_sync_lds();

    // ---- operands ------------------------------------------------------------
    // q~ = q 2^(G - M), k~ = k 2^(M - G) with G relative to the block start
    // (G2 - (M - E_I-1) = G_abs - M); q0 = q~ 2^M, k^ = k~ 2^(G_last - M),
    // kt = k~ 2^(E_I - M).  One K=32 half at a time keeps few registers live.
    QK::Vec qd[2];          // q~ in the input dtype (diagonal and, rescaled, off-diagonal blocks)
    MV q0b[2];
    // Diagonal block of A, with q~ and k~ each split into a hi and a lo part
    // in the input dtype (x = hi + lo to ~2^-16): A_II = hi.hi + lo.hi +
    // hi.lo.  Its entries are the chunk's largest (undecayed), and a single
    // bf16 rounding of both operands left o's RMS error at 3.3e-3 of its RMS
    // against 2.35e-3 for the reference's fp32 diagonal sub-chunks
    // (ops/gla/chunk.py:112-176) on the same inputs; with the split the two
    // agree.  Off-diagonal blocks are decayed and stay single products.
    f32x4 dg = (f32x4){0.f, 0.f, 0.f, 0.f};
    auto operand_half = [&](const int jj) {
      const f32x8 half = *reinterpret_cast<const f32x8 *>(&sm.fac[wv][kFacHalf][32 * jj + kq]);
      const f32x8 qf = M::widen(from_bits<MV>(cur.q[jj]));
      const f32x8 kf = M::widen(from_bits<MV>(cur.k[jj]));
      f32x8 eq, ek;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = clamp_exp(gs[jj][e] - half[e]);
        eq[e] = fast_exp2(x);
        ek[e] = fast_exp2(-x);
      }
      const f32x8 qt = qf * eq, kt = kf * ek;
      qd[jj] = QK::cvt(qt);
      const QK::Vec kd = QK::cvt(kt);
      const QK::Vec ql = QK::cvt(qt - QK::widen(qd[jj]));
      const QK::Vec kl = QK::cvt(kt - QK::widen(kd));
      dg = QK::mma(kd, qd[jj], dg);
      dg = QK::mma(kl, qd[jj], dg);
      dg = QK::mma(kd, ql, dg);
      q0b[jj] = M::cvt(qt * *reinterpret_cast<const f32x8 *>(&sm.fac[wv][kFacQ0][32 * jj + kq]));
      tile_store8(sm.kh, row, 32 * jj + kq,
                  to_bits(M::cvt(kt * *reinterpret_cast<const f32x8 *>(&sm.fac[wv][kFacKh][32 * jj + kq]))));
      tile_store8(sm.kt, row, 32 * jj + kq,
                  to_bits(QK::cvt(kt * *reinterpret_cast<const f32x8 *>(&sm.fac[wv][kFacKt][32 * jj + kq]))));
    };
    operand_half(0);
    __builtin_amdgcn_sched_barrier(0);
    operand_half(1);
    lds_barrier();  // --------------------------------------------- barrier 2

    // ---- A^T blocks (rows j of block J, columns i of this block) ------------
    // blocks J > wv are zero, block J == wv is causally masked.
    f32x4 at[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) at[J] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int J = 0; J < 3; ++J) {
      if (J < wv) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const f32x8 fj = *reinterpret_cast<const f32x8 *>(&sm.fac[wv][kFacQJ + J][32 * jj + kq]);
          const QK::Vec aj = from_bits<QK::Vec>(tile_row8(sm.kt, 16 * J + r, 32 * jj + kq));
          const QK::Vec bj = QK::cvt(QK::widen(qd[jj]) * fj);
          at[J] = QK::mma(aj, bj, at[J]);
        }
      }
    }
    {
      // causal mask on the diagonal block (row i = r, column j = 4gq + ii)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        if (4 * gq + ii > r) dg[ii] = 0.f;
#pragma unroll
      for (int J = 0; J < 4; ++J)
        if (J == wv) at[J] = dg;
    }
    // A as the B operand of V^T A^T: K slots 0-3 <- block 2pr, 4-7 <- block 2pr+1
    MV ab[2];
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      const f32x8 av = {at[2 * pr][0], at[2 * pr][1], at[2 * pr][2], at[2 * pr][3],
                        at[2 * pr + 1][0], at[2 * pr + 1][1], at[2 * pr + 1][2], at[2 * pr + 1][3]};
      ab[pr] = M::cvt(av);
    }

    // ---- per V tile: o^T = S^T q0^T + V^T A^T, store ---------------------------
#pragma unroll
    for (int t = 0; t < NVT; ++t) {
      f32x4 oacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        oacc = M::mma(from_bits<MV>(tile_row8(sm.sth, 16 * t + r, 32 * jj + kq)), q0b[jj], oacc);
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        if (2 * pr <= wv) {
          const MV va = tr_operand<MV>(sm.vs, 32 * pr + 4 * gq, 32 * pr + 16 + 4 * gq, 16 * t, lane);
          oacc = M::mma(va, ab[pr], oacc);
        }
      }
      {
        // rows past the sequence end fall outside rs.o and are dropped
        const f32x8 o8 = {oacc[0] * a.scale, oacc[1] * a.scale, oacc[2] * a.scale, oacc[3] * a.scale,
                          0.f, 0.f, 0.f, 0.f};
        const uint4 ob = to_bits(M::cvt(o8));
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_raw_buffer_store_b64((u32x2){ob.x, ob.y}, rs.o, orow + 2 * (16 * t + 4 * gq), 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- S <- 2^(G_last) S + k^^T V for the state rows of this wavefront ------
    {
      const f32x4 sdec = *reinterpret_cast<const f32x4 *>(&sm.fac[wv][kFacDec][krow]);
      const MV ka0 = tr_operand<MV>(sm.kh, 8 * gq, 8 * gq + 4, 16 * wv, lane);
      const MV ka1 = tr_operand<MV>(sm.kh, 32 + 8 * gq, 32 + 8 * gq + 4, 16 * wv, lane);
      dec_prod *= sdec;
#pragma unroll
      for (int t = 0; t < NVT; ++t) {
        S[t] *= sdec;
        S[t] = M::mma(ka0, tr_operand<MV>(sm.vs, 8 * gq, 8 * gq + 4, 16 * t, lane), S[t]);
        S[t] = M::mma(ka1, tr_operand<MV>(sm.vs, 32 + 8 * gq, 32 + 8 * gq + 4, 16 * t, lane), S[t]);
      }
    }
  };
  int c = a.c_beg;
  for (; c + 1 < a.c_end; c += 2) {
    chunk_step(buf, buf2, c);
    chunk_step(buf2, buf, c + 1);
  }
  if (c < a.c_end) chunk_step(buf, buf2, c);

  // ---- final state of the sequence -----------------------------------------
  if (a.seg == a.P - 1 && a.ht) {
    if (a.seg > 0) {
      // the lo halves of the earlier segments' states, folded as the hi
      // halves were and carried through this segment's decay
      const int64_t chain = static_cast<int64_t>(a.n) * H + h;
      f32x4 lo[NVT];
      fold_slots<NVT, true>(a, chain * a.P * KD * V + slot_index<NVT>(a.v0, wv, lane),
                            a.ws_decay + chain * a.P * KD + krow, lo);
#pragma unroll
      for (int t = 0; t < NVT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[t][i] = fmaf(dec_prod[i], lo[t][i], S[t][i]);
    }
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) a.ht[(sbase + krow + i) * V + v0 + 16 * t + r] = S[t][i];
  }
}

template <int DT, bool GF32, int NVT>
__global__ __launch_bounds__(256, SSLA_GC_SEG_WAVES) void gla_chunk_segment_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, const void *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int64_t T, int H, int V, float scale,
    const float *__restrict__ h0, uint16_t *__restrict__ o, float *__restrict__ ht, int P,
    const uint16_t *__restrict__ ws_state, const uint16_t *__restrict__ ws_lo, const float *__restrict__ ws_decay) {
  __shared__ SmemA sm;
  const int nvg = V / (16 * NVT);
  // block -> (segment, sequence, head, V group), segment-major: consecutive
  // blocks go to different XCDs, so each XCD runs every segment index in
  // equal shares (with the segment fastest, XCD s would run all of segment
  // s, and the one holding the last segments -- the longest folds -- would
  // carry all of their slot traffic alone: 54.8 against 48.1 us at C2)
  const int64_t chains = static_cast<int64_t>(n_seq) * H * nvg;
  int64_t b = blockIdx.x;
  ChunkArgs a;
  a.P = P;
  a.seg = static_cast<int>(b / chains);
  b %= chains;
  const int vg = static_cast<int>(b % nvg);
  b /= nvg;
  a.h = static_cast<int>(b % H);
  a.n = static_cast<int>(b / H);
  a.q = q; a.k = k; a.v = v; a.g = g; a.h0 = h0; a.o = o; a.ht = ht;
  a.ws_state = ws_state;
  a.ws_lo = ws_lo;
  a.ws_decay = ws_decay;
  a.H = H; a.V = V; a.scale = scale;
  a.v0 = vg * 16 * NVT;
  a.bos = min(max(cu_seqlens[a.n], (int64_t)0), T);
  const int64_t eos = min(max(cu_seqlens[a.n + 1], a.bos), T);
  a.len = eos - a.bos;
  segment_range(static_cast<int>((a.len + BT - 1) / BT), P, a.seg, a.c_beg, a.c_end);
  segment_loop<DT, GF32, NVT>(sm, a, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), threadIdx.x & 63);
}

// ----------------------------------------------------------- state pass --
struct __align__(16) SmemS {
  RowStage<false> rst[4];  // per-wavefront row staging (k, g)
  uint16_t kh[64 * 64];    // k 2^(G_last - G) rows
  uint16_t vs[64 * 64];    // v rows of the V group
  float tot[2][4][KD];     // per-block column sums of g, by chunk parity
  float fac[4][2][KD];     // per-wavefront per-key: G_last - E_I-1, 2^G_last
};

// State-only walk over segment seg (< P - 1) of one (sequence, head, V
// group):  S <- 2^(G_last) S + (k 2^(G_last - G))^T v  per chunk, from h0
// for segment 0 and from zero otherwise.  Writes the workspace slot and,
// for seg >= 1, the segment's total log2 decay.
template <int DT, bool GF32, int NVT>
__global__ __launch_bounds__(256, SSLA_GC_STATE_WAVES) void gla_chunk_state_kernel(
    const uint16_t *__restrict__ k, const uint16_t *__restrict__ v, const void *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int64_t T, int H, int V,
    const float *__restrict__ h0, int P, uint16_t *__restrict__ ws_state, uint16_t *__restrict__ ws_lo,
    float *__restrict__ ws_decay) {
  typedef Mfma<DT> M;
  typedef typename M::Vec MV;
  __shared__ SmemS sm;
  const int nvg = V / (16 * NVT);
  int64_t b = blockIdx.x;
  const int seg = static_cast<int>(b % (P - 1));
  b /= (P - 1);
  const int vg = static_cast<int>(b % nvg);
  b /= nvg;
  const int h = static_cast<int>(b % H);
  const int n = static_cast<int>(b / H);
  const int v0 = vg * 16 * NVT;
  const int vw = 16 * NVT;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, gq = lane >> 4, kq = 8 * gq;
  const int krow = 16 * wv + 4 * gq;
  const int row = 16 * wv + r;

  const int64_t sbase = (static_cast<int64_t>(n) * H + h) * KD;
  f32x4 S[NVT];
#pragma unroll
  for (int t = 0; t < NVT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      S[t][i] = (seg == 0 && h0) ? h0[(sbase + krow + i) * V + v0 + 16 * t + r] : 0.f;

  const int64_t bos = min(max(cu_seqlens[n], (int64_t)0), T);
  const int64_t eos = min(max(cu_seqlens[n + 1], bos), T);
  const int64_t len = eos - bos;
  int c_beg, c_end;
  segment_range(static_cast<int>((len + BT - 1) / BT), P, seg, c_beg, c_end);
  float dsum = 0.f;   // lane = key

  constexpr int gsz = GF32 ? 4 : 2;
  SeqRsrc rs;
  rs.k = seq_rsrc(k + bos * H * KD, len * H * KD * 2);
  rs.g = seq_rsrc(static_cast<const char *>(g) + bos * H * KD * gsz, len * H * KD * gsz);
  rs.v = seq_rsrc(v + bos * H * V, len * H * V * 2);
  LineOffs lo = line_offs(c_beg, wv, lane, H, h, V, v0, gsz);
  const uint32_t sq = BT * H * KD * 2, sg = BT * H * KD * gsz, sv = BT * H * V * 2;
  const bool vcol_ok = 8 * (lane & 7) < vw;
  // Loads run one chunk ahead over two register sets used in turn (the loop
  // is unrolled by two, so no copies).
  LineRegs buf, buf2;
  load_lines<false, GF32>(buf, rs, c_beg < c_end, lo, H, V, vcol_ok);
  auto chunk_step = [&](LineRegs &cl, LineRegs &nxt, const int c) __attribute__((always_inline)) {
    const int par = (c - c_beg) & 1;
    ChunkRegs cur;
    stage_rows<false, GF32>(sm.rst[wv], cl, lane, cur);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    lo.a16 += sq;
    lo.g += sg;
    lo.v += sv;
    load_lines<false, GF32>(nxt, rs, c + 1 < c_end, lo, H, V, vcol_ok);
    __builtin_amdgcn_sched_barrier(0);
    f32x8 gs[2];
    unpack_gates<DT, GF32>(cur, gs);
    row_scan16(gs);
    if (r == 15) {
      *reinterpret_cast<f32x8 *>(&sm.tot[par][wv][kq]) = gs[0];
      *reinterpret_cast<f32x8 *>(&sm.tot[par][wv][32 + kq]) = gs[1];
    }
    lds_barrier();  // ------------------- barrier 1 (totals ready; kh, vs free)
    {
      // lane = key: G_last - E_(wv-1) and 2^G_last
      const int kk = lane;
      const float E0 = sm.tot[par][0][kk];
      const float E1 = E0 + sm.tot[par][1][kk];
      const float E2 = E1 + sm.tot[par][2][kk];
      const float E3 = E2 + sm.tot[par][3][kk];
      const float Ep = wv == 0 ? 0.f : wv == 1 ? E0 : wv == 2 ? E1 : E2;
      sm.fac[wv][0][kk] = E3 - Ep;
      sm.fac[wv][1][kk] = fast_exp2(clamp_exp(E3));
      if (wv == 0 && seg > 0) dsum += E3;
    }
    store_v_lines(sm.vs, cl, wv, lane, vw);
    wave_sync_lds();
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const f32x8 lg = *reinterpret_cast<const f32x8 *>(&sm.fac[wv][0][32 * jj + kq]);
      f32x8 e2;
#pragma unroll
      for (int e = 0; e < 8; ++e) e2[e] = fast_exp2(clamp_exp(lg[e] - gs[jj][e]));
      const f32x8 kf = M::widen(from_bits<MV>(cur.k[jj]));
      tile_store8(sm.kh, row, 32 * jj + kq, to_bits(M::cvt(kf * e2)));
    }
    const f32x4 sdec = *reinterpret_cast<const f32x4 *>(&sm.fac[wv][1][krow]);
    lds_barrier();  // ------------------------------ barrier 2 (k^, V ready)
    const MV ka0 = tr_operand<MV>(sm.kh, 8 * gq, 8 * gq + 4, 16 * wv, lane);
    const MV ka1 = tr_operand<MV>(sm.kh, 32 + 8 * gq, 32 + 8 * gq + 4, 16 * wv, lane);
#pragma unroll
    for (int t = 0; t < NVT; ++t) {
      S[t] *= sdec;
      S[t] = M::mma(ka0, tr_operand<MV>(sm.vs, 8 * gq, 8 * gq + 4, 16 * t, lane), S[t]);
      S[t] = M::mma(ka1, tr_operand<MV>(sm.vs, 32 + 8 * gq, 32 + 8 * gq + 4, 16 * t, lane), S[t]);
    }
    // kh / vs / fac are rewritten after the next chunk's barrier 1, which
    // every wavefront reaches only after these reads
  };
  // Main loop over whole pairs (no branch between the two steps, so each
  // step's wait covers exactly its own chunk), then the odd last chunk.
  int c = c_beg;
  for (; c + 1 < c_end; c += 2) {
    chunk_step(buf, buf2, c);
    chunk_step(buf2, buf, c + 1);
  }
  if (c < c_end) chunk_step(buf, buf2, c);

  const int64_t slot = (static_cast<int64_t>(n) * H + h) * P + seg;
  const int64_t so = slot * KD * V + slot_index<NVT>(v0, wv, lane);
#pragma unroll
  for (int t = 0; t < NVT; ++t) {
    const f32x8 s8 = {S[t][0], S[t][1], S[t][2], S[t][3], 0.f, 0.f, 0.f, 0.f};
    const bf16x8 hi = QK::cvt(s8);
    const uint4 bits = to_bits(hi);
    const uint4 lbits = to_bits(QK::cvt(s8 - QK::widen(hi)));   // S - hi is exact in fp32
    *reinterpret_cast<uint2 *>(ws_state + so + 4 * t) = make_uint2(bits.x, bits.y);
    *reinterpret_cast<uint2 *>(ws_lo + so + 4 * t) = make_uint2(lbits.x, lbits.y);
  }
  if (wv == 0 && v0 == 0) ws_decay[slot * KD + lane] = dsum;
}

// Longest sequence of cu_seqlens (clamped to [0, T] as the kernels clamp
// them) against max_rows; reads cu_seqlens back in pieces of 512 entries.
int check_seq_lengths(const int64_t *cu, int n_seq, int64_t T, int64_t max_rows, hipStream_t st) {
  constexpr int kPiece = 512;
  int64_t buf[kPiece + 1];
  int64_t prev = 0;
  for (int i0 = 0; i0 <= n_seq; i0 += kPiece) {
    const int cnt = std::min(kPiece, n_seq + 1 - i0);
    const hipError_t e = read_to_host(buf, cu + i0, sizeof(int64_t) * cnt, st);
    if (e != hipSuccess) {
      set_error("gla_chunk_fwd: reading cu_seqlens failed: %s", hipGetErrorString(e));
      return SSLA_ERR_LAUNCH;
    }
    for (int j = 0; j < cnt; ++j) {
      const int64_t b = std::min(std::max(buf[j], int64_t{0}), T);
      if (i0 + j > 0) {
        const int64_t len = b - std::min(std::max(prev, int64_t{0}), T);
        if (len > max_rows) {
          set_error("gla_chunk_fwd: sequence %d has %lld rows; one sequence must stay below 2^31 bytes per "
                    "tensor (at most %lld rows at this H, K, V)", i0 + j - 1, (long long)len, (long long)max_rows);
          return SSLA_ERR_UNSUPPORTED;
        }
      }
      prev = buf[j];
    }
  }
  return SSLA_OK;
}

inline int pick_nvt(int V) {
  const int tiles = V / 16;
  for (int nvt = 4; nvt >= 1; --nvt)
    if (tiles % nvt == 0) return nvt;
  return 1;
}

// Segments per sequence: about two workgroups per CU (256 CUs), at least
// two chunks per segment on average, at most 64 segments, and a count that
// leaves no segment empty (P = ceil(chunks / ceil(chunks / P))).
inline int pick_segments(int n_seq, int64_t T, int H, int V) {
  const int nvg = V / (16 * pick_nvt(V));
  const int64_t chains = static_cast<int64_t>(n_seq) * H * nvg;
  if (chains <= 0) return 1;
  int64_t p = (512 + chains - 1) / chains;
  const int64_t avg_chunks = (T / std::max<int64_t>(n_seq, 1) + BT - 1) / BT;
  p = std::min<int64_t>(p, std::max<int64_t>(1, avg_chunks / 2));
  p = std::min<int64_t>(p, 64);
  p = std::max<int64_t>(p, 1);
  if (avg_chunks > 0) {
    const int64_t per = (avg_chunks + p - 1) / p;
    p = (avg_chunks + per - 1) / per;
  }
  return static_cast<int>(p);
}

inline size_t workspace_bytes_for(int n_seq, int H, int V, int P) {
  if (P <= 1) return 0;
  const size_t slots = static_cast<size_t>(n_seq) * H * P;
  return 2 * slots * KD * V * sizeof(uint16_t) + slots * KD * sizeof(float);   // hi, lo, decays
}

template <int DT, bool GF32, int NVT>
int launch_nvt(const void *q, const void *k, const void *v, const void *g, const int64_t *cu, int n_seq,
               int64_t T, int H, int V, float scale, const float *h0, void *o, float *ht, int P,
               uint16_t *ws_state, uint16_t *ws_lo, float *ws_decay, hipStream_t st) {
  const int nvg = V / (16 * NVT);
  const int64_t blocks_a = static_cast<int64_t>(n_seq) * H * nvg * P;
  if (blocks_a > 0x7fffffff) {
    set_error("gla_chunk_fwd: too many workgroups");
    return SSLA_ERR_UNSUPPORTED;
  }
  const uint16_t *q16 = static_cast<const uint16_t *>(q);
  uint16_t *o16 = static_cast<uint16_t *>(o);
  if (P > 1) {
    const int64_t blocks_s = static_cast<int64_t>(n_seq) * H * nvg * (P - 1);
    hipLaunchKernelGGL((gla_chunk_state_kernel<DT, GF32, NVT>), dim3(static_cast<unsigned>(blocks_s)),
                       dim3(256), 0, st, static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v),
                       g, cu, n_seq, T, H, V, h0, P, ws_state, ws_lo, ws_decay);
  }
  hipLaunchKernelGGL((gla_chunk_segment_kernel<DT, GF32, NVT>), dim3(static_cast<unsigned>(blocks_a)),
                     dim3(256), 0, st, q16, static_cast<const uint16_t *>(k),
                     static_cast<const uint16_t *>(v), g, cu, n_seq, T, H, V, scale, h0, o16, ht, P,
                     ws_state, ws_lo, ws_decay);
  return launch_status("gla_chunk_fwd");
}

template <int DT, bool GF32>
int launch_chunk(const void *q, const void *k, const void *v, const void *g, const int64_t *cu, int n_seq,
                 int64_t T, int H, int V, float scale, const float *h0, void *o, float *ht, int P,
                 uint16_t *ws_state, uint16_t *ws_lo, float *ws_decay, hipStream_t st) {
  switch (pick_nvt(V)) {
    case 4: return launch_nvt<DT, GF32, 4>(q, k, v, g, cu, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_lo, ws_decay, st);
    case 3: return launch_nvt<DT, GF32, 3>(q, k, v, g, cu, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_lo, ws_decay, st);
    case 2: return launch_nvt<DT, GF32, 2>(q, k, v, g, cu, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_lo, ws_decay, st);
    default: return launch_nvt<DT, GF32, 1>(q, k, v, g, cu, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_lo, ws_decay, st);
  }
}

}  // namespace
}  // namespace ssla

extern "C" size_t ssla_gla_chunk_workspace_size(int n_seq, int64_t T, int H, int K, int V) {
  if (n_seq <= 0 || T < 0 || H <= 0 || K != ssla::KD || V <= 0 || V % 16 != 0) return 0;
  return ssla::workspace_bytes_for(n_seq, H, V, ssla::pick_segments(n_seq, T, H, V));
}

extern "C" int ssla_gla_chunk_fwd(const void *q, const void *k, const void *v, const void *g,
                                  int g_dtype, const int64_t *cu_seqlens, int n_seq, int64_t T,
                                  int H, int K, int V, float scale, const float *h0, void *o,
                                  float *ht, int dtype, void *workspace, size_t workspace_bytes,
                                  void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && T >= 0 && H > 0 && K > 0 && V > 0,
                 "gla_chunk_fwd: bad sizes n_seq=%d T=%lld H=%d K=%d V=%d", n_seq, (long long)T, H, K, V);
  if (K != KD || V % 16 != 0 || V > 256) {
    set_error("gla_chunk_fwd: needs K == 64 and V a multiple of 16 up to 256 (K=%d V=%d)", K, V);
    return SSLA_ERR_UNSUPPORTED;
  }
  if (n_seq == 0) return SSLA_OK;
  SSLA_CHECK_ARG(cu_seqlens != nullptr, "gla_chunk_fwd: cu_seqlens is NULL");
  // kernels address a sequence with 32-bit byte offsets
  {
    // Each sequence's rows are addressed through buffer resources with
    // 32-bit byte offsets: a sequence must stay below 2^31 bytes per tensor.
    // Only a batch whose whole tensor reaches that size can hold such a
    // sequence; then the lengths are read back (one host synchronisation).
    const int64_t row_bytes = static_cast<int64_t>(H) * std::max(K, V) * 4;
    const int64_t max_rows = ((int64_t{1} << 31) - 1) / row_bytes;
    if (T > max_rows) {
      const int st = check_seq_lengths(cu_seqlens, n_seq, T, max_rows, static_cast<hipStream_t>(stream));
      if (st != SSLA_OK) return st;
    }
  }
  SSLA_CHECK_ARG(T == 0 || (q && k && v && g && o), "gla_chunk_fwd: null tensor pointer");
  SSLA_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(g, 16) && aligned(v, 16) && aligned(o, 8),
                 "gla_chunk_fwd: q/k/g/v must be 16-byte and o 8-byte aligned");
  if (dtype != SSLA_BF16 && dtype != SSLA_F16) {
    set_error("gla_chunk_fwd: dtype %d not supported (bf16 or fp16)", dtype);
    return SSLA_ERR_DTYPE;
  }
  if (g_dtype != SSLA_F32 && g_dtype != dtype) {
    set_error("gla_chunk_fwd: g dtype %d must be fp32 or the dtype of q", g_dtype);
    return SSLA_ERR_DTYPE;
  }
  const int P = pick_segments(n_seq, T, H, V);
  const size_t need = workspace_bytes_for(n_seq, H, V, P);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("gla_chunk_fwd: workspace of %zu bytes needed (ssla_gla_chunk_workspace_size), %zu given",
              need, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(need == 0 || aligned(workspace, 16), "gla_chunk_fwd: workspace must be 16-byte aligned");
  uint16_t *ws_state = static_cast<uint16_t *>(workspace);
  // slots are K*V*2 bytes (a multiple of 2048), so lo and the decays stay 16-byte aligned
  const size_t slot_elems = static_cast<size_t>(n_seq) * H * P * KD * V;
  uint16_t *ws_lo = need ? ws_state + slot_elems : nullptr;
  float *ws_decay = need ? reinterpret_cast<float *>(ws_state + 2 * slot_elems) : nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool gf32 = g_dtype == SSLA_F32;
  if (dtype == SSLA_BF16)
    return gf32 ? launch_chunk<SSLA_BF16, true>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_lo, ws_decay, st)
                : launch_chunk<SSLA_BF16, false>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_lo, ws_decay, st);
  return gf32 ? launch_chunk<SSLA_F16, true>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_lo, ws_decay, st)
              : launch_chunk<SSLA_F16, false>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_lo, ws_decay, st);
}

namespace ssla {
namespace {

constexpr int kMaxScratchDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the device that runs `stream` (the current
// device for the null stream), looked up once per device with that device
// current and cached.
int noalloc_scratch(hipStream_t stream, void **out) {
  int cur = 0, dev = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess) {
    dev = cur;
    if (stream) e = hipStreamGetDevice(stream, &dev);
  }
  if (e != hipSuccess) {
    set_error("gla_chunk_fwd_noalloc: device query failed: %s", hipGetErrorString(e));
    return SSLA_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) {
    set_error("gla_chunk_fwd_noalloc: device %d beyond the %d the scratch table holds", dev, kMaxScratchDevices);
    return SSLA_ERR_UNSUPPORTED;
  }
  void *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      if (dev != cur) e = hipSetDevice(dev);
      if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (dev != cur) {
        const hipError_t e2 = hipSetDevice(cur);
        if (e == hipSuccess) e = e2;
      }
      if (e != hipSuccess || p == nullptr) {
        set_error("gla_chunk_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
        return SSLA_ERR_LAUNCH;
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return SSLA_OK;
}

}  // namespace
}  // namespace ssla

extern "C" int ssla_gla_chunk_fwd_noalloc(const void *q, const void *k, const void *v, const void *g,
                                          int g_dtype, const int64_t *cu_seqlens, int n_seq, int64_t T,
                                          int H, int K, int V, float scale, const float *h0, void *o,
                                          float *ht, int dtype, void *stream) {
  using namespace ssla;
  clear_error();
  const size_t need = ssla_gla_chunk_workspace_size(n_seq, T, H, K, V);
  if (need > kNoallocScratchBytes) {
    set_error("gla_chunk_fwd_noalloc: this shape needs %zu bytes of workspace, the static scratch holds %zu "
              "(call ssla_gla_chunk_fwd with a workspace)", need, kNoallocScratchBytes);
    return SSLA_ERR_WORKSPACE;
  }
  void *ws = nullptr;
  if (need > 0) {
    const int st = noalloc_scratch(static_cast<hipStream_t>(stream), &ws);
    if (st != SSLA_OK) return st;
  }
  return ssla_gla_chunk_fwd(q, k, v, g, g_dtype, cu_seqlens, n_seq, T, H, K, V, scale, h0, o, ht, dtype, ws,
                            need > 0 ? kNoallocScratchBytes : 0, stream);
}
