// Chunked gated-linear-attention forward, fused into one launch (gfx950).
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
// Design:
// * One workgroup (4 wavefronts) owns one (sequence, head, 16-column V
//   tile) and walks the chunks of its sequence serially.  The fp32 state
//   tile S[64 x 16] never leaves the chip: wavefront w keeps rows
//   16w..16w+15 as an MFMA accumulator, and a transposed copy sits in LDS
//   for the other wavefronts.  Nothing but q, k, v, g, h0 is read and
//   nothing but o, ht is written: g's cumsum, A and the per-chunk states of
//   the reference never reach HBM.
// * The V tiles of one (sequence, head) are placed on the same XCD (the
//   hardware deals workgroups round-robin over the 8 XCDs), so the q, k, g
//   they share come from that XCD's L2 after the first reader.
// * Wavefront I owns the 16 chunk rows 16I..16I+15 ("block" I).  All
//   products use v_mfma_f32_16x16x32_{bf16,f16}.  Within a lane the 64 keys
//   are held as k = 32*jj + 8*(lane/16) + e (jj = 0,1; e = 0..7), which is
//   the operand layout of the two K=32 halves of a K=64 product.
// * Decay factorisation (log2 units, G2 = G * log2(e)): with R_J = G2 at the
//   end of block J-1 (R_0 = 0),
//     exp(G_i - G_j) = 2^(G2_i - R_J) * 2^(R_J - G2_j)      (j in block J).
//   The first factor is <= 1 for i in a later or the same block, the second
//   grows by at most the decay of the 16 rows of block J.  A chunk whose
//   gates leave that range (a block decay below -64 in log2 units, or any
//   positive log-gate) is computed in "exact" mode instead: the diagonal
//   blocks elementwise and the off-diagonal blocks re-referenced to the row
//   block, as the reference does (ops/gla/chunk.py:80-92, :160-166).
//   Exact mode is chosen per chunk, uniformly for the workgroup.
// * The state enters the output product split into bf16 high and low parts,
//   so S contributes with ~16 mantissa bits (the reference rounds its
//   per-chunk states to bf16, ops/gla/chunk.py:933).
#include "common.h"

namespace ssla {
namespace {

constexpr int BT = 64;    // chunk rows
constexpr int KD = 64;    // key width
constexpr int BV = 16;    // value columns per workgroup
constexpr float kGrowthLimit = 64.f;   // log2 units

// LDS row pitches (elements); padding breaks power-of-two bank strides.
constexpr int kSP = KD + 4;    // S^T rows: [v][k] fp32
constexpr int kKP = KD + 8;    // K-tilde rows: [j][k] 16-bit
constexpr int kTP = BT + 8;    // transposed rows: [k][j] / [v][j] 16-bit
constexpr int kXP = KD + 4;    // exact-mode G rows: [j][k] fp32

typedef float f32x8 __attribute__((ext_vector_type(8)));

// MFMA of the input dtype (value products: S q~, A v, k~s^T v).
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
// holds the growth factor 2^(R_J - G2_j) (up to 2^64) that fp16 cannot.
typedef Mfma<SSLA_BF16> QK;

template <class V8>
__device__ __forceinline__ V8 from_bits(const uint4 &x) { return __builtin_bit_cast(V8, x); }
template <class V8>
__device__ __forceinline__ uint4 to_bits(const V8 &x) { return __builtin_bit_cast(uint4, x); }

struct __align__(16) Smem {
  float st[2][BV][kSP];          // S^T, double-buffered by chunk parity
  uint16_t kt[4][16][kKP];       // bf16 K-tilde of block J (row j, key k)
  uint16_t kst[KD][kTP];         // K-state transposed (key k, row j), input dtype
  uint16_t vt[BV][kTP];          // V tile transposed (column v, row j)
  float tot[4][KD];              // per-block column sums of g (log2 units)
  float fac[4][7][KD];           // per-wavefront per-key factors (see below)
  int flag[4];                   // per-wavefront "needs exact mode"
  // exact mode only
  uint16_t xq[BT][kKP];          // raw q rows (input dtype)
  uint16_t xk[BT][kKP];          // raw k rows (input dtype)
  float xg[BT][kXP];             // G2 rows
};
// fac[I][.] slots, lane = key:  0: R_I   1: 2^(G_last - R_I)   2: 2^(G_last)
//                                3: G_last   4 + J: 2^(R_I - R_J) for J < I
constexpr int kFacR = 0, kFacState = 1, kFacDecay = 2, kFacLast = 3, kFacJ0 = 4;

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

// Raw global loads for one chunk, held across the previous chunk's compute.
struct ChunkRegs {
  uint4 q[2], k[2];   // 2 x 8 keys of this lane's row (16-bit)
  float4 g[4];        // 16 log-gates (fp32 g) ...
  uint4 g16[2];       // ... or 16-bit g
  uint2 v;            // 4 values of one V-tile row
};

template <bool GF32>
__device__ __forceinline__ void load_chunk(ChunkRegs &R, const uint16_t *__restrict__ q,
                                           const uint16_t *__restrict__ k,
                                           const uint16_t *__restrict__ v, const void *__restrict__ g,
                                           int64_t t_row, bool row_ok, int64_t t_vrow, bool vrow_ok,
                                           int H, int V, int h, int kq, int vcol) {
  const int64_t base = (t_row * H + h) * KD;
  if (row_ok) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      R.q[jj] = *reinterpret_cast<const uint4 *>(q + base + 32 * jj + kq);
      R.k[jj] = *reinterpret_cast<const uint4 *>(k + base + 32 * jj + kq);
      if (GF32) {
        const float *gp = static_cast<const float *>(g) + base + 32 * jj + kq;
        R.g[2 * jj] = *reinterpret_cast<const float4 *>(gp);
        R.g[2 * jj + 1] = *reinterpret_cast<const float4 *>(gp + 4);
      } else {
        R.g16[jj] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(g) + base + 32 * jj + kq);
      }
    }
  } else {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      R.q[jj] = make_uint4(0, 0, 0, 0);
      R.k[jj] = make_uint4(0, 0, 0, 0);
      R.g[2 * jj] = make_float4(0.f, 0.f, 0.f, 0.f);
      R.g[2 * jj + 1] = make_float4(0.f, 0.f, 0.f, 0.f);
      R.g16[jj] = make_uint4(0, 0, 0, 0);
    }
  }
  R.v = vrow_ok ? *reinterpret_cast<const uint2 *>(v + (t_vrow * H + h) * V + vcol) : make_uint2(0, 0);
}

// 16 per-key values of this lane's key set from an LDS row of 64.
__device__ __forceinline__ void lds_keys(const float *row, int kq, f32x8 out[2]) {
  out[0] = *reinterpret_cast<const f32x8 *>(row + kq);
  out[1] = *reinterpret_cast<const f32x8 *>(row + 32 + kq);
}

struct ChunkArgs {
  const uint16_t *q, *k, *v;
  const void *g;
  const float *h0;
  uint16_t *o;
  float *ht;
  int64_t bos, len;
  int H, V, h, n, v0;
  float scale;
};

// The chunk loop of wavefront I (rows 16I..16I+15 of every chunk).  I is a
// template parameter so that all block-dependent indexing is static; the
// four wavefronts run different instantiations and meet at the same
// hardware barriers (two per chunk).
template <int DT, bool GF32, int I>
__device__ __forceinline__ void chunk_loop(Smem &sm, const ChunkArgs &a, int lane) {
  typedef Mfma<DT> M;
  typedef typename M::Vec MV;
  const int r = lane & 15;        // row within block / MFMA column index
  const int gq = lane >> 4;       // lane group
  const int kq = 8 * gq;          // key offset of this lane inside each K=32 half
  const int H = a.H, V = a.V, h = a.h, v0 = a.v0;
  const int64_t len = a.len;
  const int nchunks = static_cast<int>((len + BT - 1) / BT);

  // ---- initial state: rows 16I + 4gq + i, column v0 + r -------------------
  const int64_t sbase = (static_cast<int64_t>(a.n) * H + h) * KD;
  f32x4 S;
#pragma unroll
  for (int i = 0; i < 4; ++i) S[i] = a.h0 ? a.h0[(sbase + 16 * I + 4 * gq + i) * V + v0 + r] : 0.f;
  *reinterpret_cast<f32x4 *>(&sm.st[0][r][16 * I + 4 * gq]) = S;

  // V-tile row handled by this lane when staging V: row 16I + lane/4, columns 4*(lane%4)..+3
  const int vrow = 16 * I + (lane >> 2);
  const int vcol = v0 + 4 * (lane & 3);
  const int row = 16 * I + r;

  ChunkRegs nxt;
  if (nchunks > 0)
    load_chunk<GF32>(nxt, a.q, a.k, a.v, a.g, a.bos + row, row < len, a.bos + vrow, vrow < len, H, V, h,
                     kq, vcol);

  for (int c = 0; c < nchunks; ++c) {
    const int cur = c & 1;
    const int64_t t0 = a.bos + static_cast<int64_t>(c) * BT;
    const int64_t rem = len - static_cast<int64_t>(c) * BT;   // valid rows in this chunk (>0)
    ChunkRegs R = nxt;
    if (c + 1 < nchunks) {
      const int64_t rem2 = rem - BT;
      load_chunk<GF32>(nxt, a.q, a.k, a.v, a.g, t0 + BT + row, row < rem2, t0 + BT + vrow, vrow < rem2,
                       H, V, h, kq, vcol);
    }

    // ---- unpack: element e of half jj is key 32*jj + kq + e ---------------
    f32x8 qf[2], kf[2], gs[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      qf[jj] = M::widen(from_bits<MV>(R.q[jj]));
      kf[jj] = M::widen(from_bits<MV>(R.k[jj]));
      if (GF32) {
        const f32x4 x0 = __builtin_bit_cast(f32x4, R.g[2 * jj]), x1 = __builtin_bit_cast(f32x4, R.g[2 * jj + 1]);
        gs[jj] = (f32x8){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]} * kLog2e;
      } else {
        gs[jj] = M::widen(from_bits<MV>(R.g16[jj])) * kLog2e;
      }
    }
    // positive log-gates are outside the factorised path
    float gmax = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int e = 0; e < 8; ++e) gmax = fmaxf(gmax, gs[jj][e]);
    // ---- block-local inclusive cumsum over the 16 rows (DPP row scan) ------
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int e = 0; e < 8; ++e) gs[jj][e] = row_inclusive_scan(gs[jj][e]);
    float smin = INFINITY;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int e = 0; e < 8; ++e) smin = fminf(smin, gs[jj][e]);
    const bool need_exact = gmax > 0.f || smin < -kGrowthLimit;
    if (r == 15) {
      *reinterpret_cast<f32x8 *>(&sm.tot[I][kq]) = gs[0];
      *reinterpret_cast<f32x8 *>(&sm.tot[I][32 + kq]) = gs[1];
    }
    const bool wflag = __builtin_amdgcn_ballot_w64(need_exact) != 0;
    if (lane == 0) sm.flag[I] = wflag ? 1 : 0;
    lds_barrier();  // --------------------------------------------- barrier 1
    const bool exact = (sm.flag[0] | sm.flag[1] | sm.flag[2] | sm.flag[3]) != 0;

    // ---- per-key references and factors (lane = key) -----------------------
    {
      const int kk = lane;
      float ref[5];
      ref[0] = 0.f;
#pragma unroll
      for (int J = 0; J < 4; ++J) ref[J + 1] = ref[J] + sm.tot[J][kk];
      sm.fac[I][kFacR][kk] = ref[I];                               // R_I
      sm.fac[I][kFacState][kk] = fast_exp2(ref[4] - ref[I]);       // 2^(G_last - R_I)
      sm.fac[I][kFacDecay][kk] = fast_exp2(ref[4]);                // 2^(G_last)
      sm.fac[I][kFacLast][kk] = ref[4];                            // G_last
#pragma unroll
      for (int J = 0; J < I; ++J) sm.fac[I][kFacJ0 + J][kk] = fast_exp2(ref[I] - ref[J]);  // 2^(R_I - R_J)
    }
    wave_sync_lds();
    f32x8 offs[2], fstate[2];
    lds_keys(sm.fac[I][kFacR], kq, offs);
    lds_keys(sm.fac[I][kFacState], kq, fstate);
    // own-row decays of the state rows 16I + 4gq + i
    const f32x4 sdec = *reinterpret_cast<const f32x4 *>(&sm.fac[I][kFacDecay][16 * I + 4 * gq]);

    // ---- operands of this block ------------------------------------------
    // qt = q * 2^(G2_i - R_I) * scale (fp32, kept for the re-referenced copies)
    f32x8 qt[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      f32x8 e2;
#pragma unroll
      for (int e = 0; e < 8; ++e) e2[e] = fast_exp2(gs[jj][e]);
      qt[jj] = qf[jj] * e2 * a.scale;
    }
    {
      f32x8 kt[2], ks[2];
      if (!exact) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          f32x8 e2;
#pragma unroll
          for (int e = 0; e < 8; ++e) e2[e] = fast_exp2(-gs[jj][e]);
          kt[jj] = kf[jj] * e2;                 // 2^(R_I - G2_j)
          ks[jj] = kt[jj] * fstate[jj];         // 2^(G_last - G2_j)
        }
      } else {
        f32x8 gl[2];
        lds_keys(sm.fac[I][kFacLast], kq, gl);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          kt[jj] = (f32x8){0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          f32x8 e2;
#pragma unroll
          for (int e = 0; e < 8; ++e) e2[e] = fast_exp2(gl[jj][e] - (gs[jj][e] + offs[jj][e]));
          ks[jj] = kf[jj] * e2;
        }
      }
      *reinterpret_cast<uint4 *>(&sm.kt[I][r][kq]) = to_bits(QK::cvt(kt[0]));
      *reinterpret_cast<uint4 *>(&sm.kt[I][r][32 + kq]) = to_bits(QK::cvt(kt[1]));
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const uint4 kb = to_bits(M::cvt(ks[jj]));
        const uint32_t w4[4] = {kb.x, kb.y, kb.z, kb.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          sm.kst[32 * jj + kq + e][16 * I + r] =
              static_cast<uint16_t>((e & 1) ? (w4[e >> 1] >> 16) : (w4[e >> 1] & 0xffffu));
      }
    }
    sm.vt[4 * (lane & 3) + 0][vrow] = static_cast<uint16_t>(R.v.x & 0xffffu);
    sm.vt[4 * (lane & 3) + 1][vrow] = static_cast<uint16_t>(R.v.x >> 16);
    sm.vt[4 * (lane & 3) + 2][vrow] = static_cast<uint16_t>(R.v.y & 0xffffu);
    sm.vt[4 * (lane & 3) + 3][vrow] = static_cast<uint16_t>(R.v.y >> 16);
    if (exact) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        *reinterpret_cast<uint4 *>(&sm.xq[16 * I + r][32 * jj + kq]) = R.q[jj];
        *reinterpret_cast<uint4 *>(&sm.xk[16 * I + r][32 * jj + kq]) = R.k[jj];
        *reinterpret_cast<f32x8 *>(&sm.xg[16 * I + r][32 * jj + kq]) = gs[jj] + offs[jj];
      }
    }
    lds_barrier();  // --------------------------------------------- barrier 2

    // ---- o^T = S^T (q~)^T  +  V^T A^T  (MFMA rows = v, columns = i) --------
    // q referenced to the chunk start (R_0 = 0): q~0 = qt * 2^(R_I)
    f32x8 q0[2];
    if (I == 0) {
      q0[0] = qt[0];
      q0[1] = qt[1];
    } else {
      f32x8 f0[2];
      lds_keys(sm.fac[I][kFacJ0], kq, f0);
      q0[0] = qt[0] * f0[0];
      q0[1] = qt[1] * f0[1];
    }
    f32x4 oacc = {0.f, 0.f, 0.f, 0.f};
    {
      const MV qb0 = M::cvt(q0[0]), qb1 = M::cvt(q0[1]);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const f32x8 sv = *reinterpret_cast<const f32x8 *>(&sm.st[cur][r][32 * jj + kq]);
        const MV shi = M::cvt(sv);
        const MV slo = M::cvt(sv - M::widen(shi));
        const MV qb = jj ? qb1 : qb0;
        oacc = M::mma(shi, qb, oacc);
        oacc = M::mma(slo, qb, oacc);
      }
    }

    // A^T blocks (rows j of block J, columns i of this block)
    f32x4 at[I + 1];
#pragma unroll
    for (int J = 0; J <= I; ++J) at[J] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (!exact) {
#pragma unroll
      for (int J = 0; J <= I; ++J) {
        // q re-referenced to R_J: qt * 2^(R_I - R_J)
        f32x8 qj[2];
        if (J == I) {
          qj[0] = qt[0];
          qj[1] = qt[1];
        } else if (J == 0) {
          qj[0] = q0[0];
          qj[1] = q0[1];
        } else {
          f32x8 fj[2];
          lds_keys(sm.fac[I][kFacJ0 + J], kq, fj);
          qj[0] = qt[0] * fj[0];
          qj[1] = qt[1] * fj[1];
        }
        const QK::Vec a0 = from_bits<QK::Vec>(*reinterpret_cast<const uint4 *>(&sm.kt[J][r][kq]));
        const QK::Vec a1 = from_bits<QK::Vec>(*reinterpret_cast<const uint4 *>(&sm.kt[J][r][32 + kq]));
        at[J] = QK::mma(a0, QK::cvt(qj[0]), at[J]);
        at[J] = QK::mma(a1, QK::cvt(qj[1]), at[J]);
      }
    } else {
      // off-diagonal blocks: k re-referenced to R_I (<= 1 for decays)
#pragma unroll
      for (int J = 0; J < I; ++J) {
        const int jrow = 16 * J + r;
        f32x8 kj[2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const f32x8 kr = M::widen(from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.xk[jrow][32 * jj + kq])));
          const f32x8 gr = *reinterpret_cast<const f32x8 *>(&sm.xg[jrow][32 * jj + kq]);
          f32x8 e2;
#pragma unroll
          for (int e = 0; e < 8; ++e) e2[e] = fast_exp2(offs[jj][e] - gr[e]);
          kj[jj] = kr * e2;
        }
        at[J] = QK::mma(QK::cvt(kj[0]), QK::cvt(qt[0]), at[J]);
        at[J] = QK::mma(QK::cvt(kj[1]), QK::cvt(qt[1]), at[J]);
      }
      // diagonal block elementwise: lane holds A[i = r][j = 4gq + ii]
      const int irow = 16 * I + r;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int j = 4 * gq + ii;
        const int jrow = 16 * I + j;
        float acc = 0.f;
        if (j <= r) {
#pragma unroll 1
          for (int k8 = 0; k8 < KD; k8 += 8) {
            const f32x8 qv = M::widen(from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.xq[irow][k8])));
            const f32x8 kv = M::widen(from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.xk[jrow][k8])));
            const f32x8 gi = *reinterpret_cast<const f32x8 *>(&sm.xg[irow][k8]);
            const f32x8 gj = *reinterpret_cast<const f32x8 *>(&sm.xg[jrow][k8]);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += qv[e] * kv[e] * fast_exp2(gi[e] - gj[e]);
          }
        }
        at[I][ii] = acc * a.scale;
      }
    }
    // causal mask on the diagonal block (row i = r, column j = 4gq + ii)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      if (4 * gq + ii > r) at[I][ii] = 0.f;

    // V^T A^T over pairs of blocks: K slots 0-3 <- block J0, 4-7 <- block J1
#pragma unroll
    for (int J0 = 0; J0 <= I; J0 += 2) {
      const int J1 = J0 + 1;
      f32x8 av;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        av[ii] = at[J0][ii];
        av[4 + ii] = J1 <= I ? at[J1 <= I ? J1 : J0][ii] : 0.f;
      }
      const uint2 va = *reinterpret_cast<const uint2 *>(&sm.vt[r][16 * J0 + 4 * gq]);
      const uint2 vb = J1 <= I ? *reinterpret_cast<const uint2 *>(&sm.vt[r][16 * J1 + 4 * gq]) : make_uint2(0, 0);
      const MV vop = from_bits<MV>(make_uint4(va.x, va.y, vb.x, vb.y));
      oacc = M::mma(vop, M::cvt(av), oacc);
    }

    // ---- store o: lane holds o[row 16I + r][v0 + 4gq .. +3] ----------------
    if (row < rem) {
      const f32x8 o8 = {oacc[0], oacc[1], oacc[2], oacc[3], 0.f, 0.f, 0.f, 0.f};
      const uint4 ob = to_bits(M::cvt(o8));
      *reinterpret_cast<uint2 *>(a.o + ((t0 + row) * H + h) * V + v0 + 4 * gq) = make_uint2(ob.x, ob.y);
    }

    // ---- state update of rows 16I..16I+15: S <- 2^(G_last) S + Ks^T V -------
    S *= sdec;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const MV ka = from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.kst[16 * I + r][32 * jj + kq]));
      const MV vb = from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.vt[r][32 * jj + kq]));
      S = M::mma(ka, vb, S);
    }
    *reinterpret_cast<f32x4 *>(&sm.st[cur ^ 1][r][16 * I + 4 * gq]) = S;
  }

  if (a.ht) {
#pragma unroll
    for (int i = 0; i < 4; ++i) a.ht[(sbase + 16 * I + 4 * gq + i) * V + v0 + r] = S[i];
  }
}

template <int DT, bool GF32>
__global__ __launch_bounds__(256, 1) void gla_chunk_fwd_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, const void *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int64_t T, int H, int V, float scale,
    const float *__restrict__ h0, uint16_t *__restrict__ o, float *__restrict__ ht) {
  __shared__ Smem sm;
  const int n_vt = V / BV;
  // ---- XCD-aware block -> (sequence*head, V tile) mapping ------------------
  // Workgroups are dealt round-robin over the 8 XCDs; consecutive linear
  // ids inside one XCD share a (sequence, head), so its V tiles share L2.
  const int64_t nblk = static_cast<int64_t>(gridDim.x);
  const int64_t b = blockIdx.x;
  const int64_t xcd = b & 7, slot = b >> 3;
  const int64_t lin = xcd * (nblk >> 3) + min(xcd, nblk & 7) + slot;
  ChunkArgs a;
  a.q = q; a.k = k; a.v = v; a.g = g; a.h0 = h0; a.o = o; a.ht = ht;
  a.H = H; a.V = V; a.scale = scale;
  const int vt = static_cast<int>(lin % n_vt);
  const int64_t sh = lin / n_vt;
  a.h = static_cast<int>(sh % H);
  a.n = static_cast<int>(sh / H);
  a.v0 = vt * BV;
  a.bos = min(max(cu_seqlens[a.n], (int64_t)0), T);
  const int64_t eos = min(max(cu_seqlens[a.n + 1], a.bos), T);
  a.len = eos - a.bos;
  const int lane = threadIdx.x & 63;
  switch (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) {
    case 0: chunk_loop<DT, GF32, 0>(sm, a, lane); break;
    case 1: chunk_loop<DT, GF32, 1>(sm, a, lane); break;
    case 2: chunk_loop<DT, GF32, 2>(sm, a, lane); break;
    default: chunk_loop<DT, GF32, 3>(sm, a, lane); break;
  }
}

template <int DT>
int launch_chunk(const void *q, const void *k, const void *v, const void *g, bool gf32,
                 const int64_t *cu, int n_seq, int64_t T, int H, int V, float scale, const float *h0,
                 void *o, float *ht, hipStream_t st) {
  const int64_t blocks = static_cast<int64_t>(n_seq) * H * (V / BV);
  if (blocks == 0) return SSLA_OK;
  if (blocks > 0x7fffffff) {
    set_error("gla_chunk_fwd: too many workgroups");
    return SSLA_ERR_UNSUPPORTED;
  }
  const uint16_t *q16 = static_cast<const uint16_t *>(q);
  const uint16_t *k16 = static_cast<const uint16_t *>(k);
  const uint16_t *v16 = static_cast<const uint16_t *>(v);
  uint16_t *o16 = static_cast<uint16_t *>(o);
  if (gf32)
    hipLaunchKernelGGL((gla_chunk_fwd_kernel<DT, true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       q16, k16, v16, g, cu, n_seq, T, H, V, scale, h0, o16, ht);
  else
    hipLaunchKernelGGL((gla_chunk_fwd_kernel<DT, false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       q16, k16, v16, g, cu, n_seq, T, H, V, scale, h0, o16, ht);
  return launch_status("gla_chunk_fwd");
}

}  // namespace
}  // namespace ssla

extern "C" int ssla_gla_chunk_fwd(const void *q, const void *k, const void *v, const void *g,
                                  int g_dtype, const int64_t *cu_seqlens, int n_seq, int64_t T,
                                  int H, int K, int V, float scale, const float *h0, void *o,
                                  float *ht, int dtype, void *workspace, size_t workspace_bytes,
                                  void *stream) {
  using namespace ssla;
  (void)workspace;
  (void)workspace_bytes;
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && T >= 0 && H > 0 && K > 0 && V > 0,
                 "gla_chunk_fwd: bad sizes n_seq=%d T=%lld H=%d K=%d V=%d", n_seq, (long long)T, H, K, V);
  if (K != KD || V % BV != 0 || V > 256) {
    set_error("gla_chunk_fwd: needs K == 64 and V a multiple of 16 up to 256 (K=%d V=%d)", K, V);
    return SSLA_ERR_UNSUPPORTED;
  }
  if (n_seq == 0) return SSLA_OK;
  SSLA_CHECK_ARG(cu_seqlens != nullptr, "gla_chunk_fwd: cu_seqlens is NULL");
  SSLA_CHECK_ARG(T == 0 || (q && k && v && g && o), "gla_chunk_fwd: null tensor pointer");
  SSLA_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(g, 16) && aligned(v, 8) && aligned(o, 8),
                 "gla_chunk_fwd: q/k/g must be 16-byte and v/o 8-byte aligned");
  if (dtype != SSLA_BF16 && dtype != SSLA_F16) {
    set_error("gla_chunk_fwd: dtype %d not supported (bf16 or fp16)", dtype);
    return SSLA_ERR_DTYPE;
  }
  if (g_dtype != SSLA_F32 && g_dtype != dtype) {
    set_error("gla_chunk_fwd: g dtype %d must be fp32 or the dtype of q", g_dtype);
    return SSLA_ERR_DTYPE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool gf32 = g_dtype == SSLA_F32;
  if (dtype == SSLA_BF16)
    return launch_chunk<SSLA_BF16>(q, k, v, g, gf32, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, st);
  return launch_chunk<SSLA_F16>(q, k, v, g, gf32, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, st);
}
