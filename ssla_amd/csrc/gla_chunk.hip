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
// Schedule (two launches; the only intermediate is one state per segment):
// * Each sequence is cut into P segments of whole chunks (P picked so that
//   about two workgroups run per CU; no work is repeated across them).
// * Kernel S ("state pass"): for segments 0..P-2, one workgroup walks the
//   chunks of its (sequence, head, segment) computing only the state update
//   (from h0 for segment 0, from zero otherwise) and leaves the final state
//   and the total log-decay in the workspace.  It reads k, g, v only.
// * Kernel A ("segment"): one workgroup per (sequence, head, segment) folds
//   the earlier segments into its entering state
//     S_e(1) = slot 0,  S_e(s+1) = 2^D(s) S_e(s) + slot s,
//   then runs the full chunk loop below and writes o (and ht for the last
//   segment).  Its k, g, v re-reads of segments 0..P-2 are served mostly by
//   the Infinity Cache right after kernel S.
//   P = 1 (no workspace) runs kernel A alone.
//
// Kernel A per chunk:
// * Wavefront I owns the 16 chunk rows 16I..16I+15 ("block" I) and the
//   state rows 16I..16I+15 (as MFMA accumulators).  All products use
//   v_mfma_f32_16x16x32_{bf16,f16}; every wavefront runs the same code,
//   block-dependent work is predicated on the (uniform) index.  Within a
//   lane the 64 keys are held as k = 32*jj + 8*(lane/16) + e (jj = 0,1;
//   e = 0..7): the operand layout of the two K=32 halves of a K=64 product.
// * Decay factorisation (log2 units, G2 = G * log2(e)): with R = G2 at the
//   middle of the chunk (end of row 31),
//     exp(G_i - G_j) = 2^(G2_i - R) * 2^(R - G2_j),
//   so every block of A uses the same two operands q~ = q 2^(G2 - R) and
//   k~ = k 2^(R - G2).  Both stay inside 2^(+-50) when neither half of the
//   chunk decays by more than 2^-50 (typical GLA gates decay ~2^-1 per row
//   per key, i.e. 2^-32 per half chunk).  A chunk outside that range, or with
//   any positive log-gate, is computed in "exact" mode: the diagonal 16x16
//   blocks elementwise and the off-diagonal blocks re-referenced to the row
//   block, as the reference does (ops/gla/chunk.py:80-92, :160-166).  The
//   mode is chosen per chunk, uniformly for the workgroup.
// * The state enters the output product split into high and low 16-bit
//   parts (written once by the wavefront that owns the rows), so S
//   contributes with ~16 mantissa bits (the reference rounds its per-chunk
//   states to bf16, ops/gla/chunk.py:933).  scale is applied to o at the end.
#include "common.h"

namespace ssla {
namespace {

constexpr int BT = 64;    // chunk rows
constexpr int KD = 64;    // key width
constexpr float kRangeLimit = 50.f;    // |G2 - R| bound of the fast path, log2 units

// LDS row pitches (elements); padding breaks power-of-two bank strides.
constexpr int kKP = KD + 8;    // [row][key] 16-bit
constexpr int kTP = BT + 8;    // transposed [key or column][row] 16-bit
constexpr int kXP = KD + 4;    // exact-mode G rows: [row][key] fp32

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
// holds the factors 2^(+-50) that fp16 cannot.
typedef Mfma<SSLA_BF16> QK;

template <class V8>
__device__ __forceinline__ V8 from_bits(const uint4 &x) { return __builtin_bit_cast(V8, x); }
template <class V8>
__device__ __forceinline__ uint4 to_bits(const V8 &x) { return __builtin_bit_cast(uint4, x); }

template <int NVT>
struct __align__(16) SmemA {
  uint16_t sth[16 * NVT][kKP];   // S^T high part (column v, key k)
  uint16_t stl[16 * NVT][kKP];   // S^T low part
  uint16_t kt[BT][kKP];          // bf16 k~ rows (fast) / raw k rows (exact)
  uint16_t kst[KD][kTP];         // k~s transposed (key k, row j), input dtype
  uint16_t vt[16 * NVT][kTP];    // V tile transposed (column v, row j)
  float tot[4][KD];              // per-block column sums of g (log2 units)
  float fac[4][6][KD];           // per-wavefront per-key values (slots below)
  int flag[4];                   // per-wavefront "saw a positive log-gate"
  uint16_t xq[BT][kKP];          // exact mode: raw q rows
  float xg[BT][kXP];             // exact mode: G2 rows
};
// fac[I][.] slots, lane = key
constexpr int kFacRel = 0;    // R_I - R         (R_I = G2 at the end of block I-1)
constexpr int kFacKs = 1;     // 2^(G_last - R)
constexpr int kFacQ0 = 2;     // 2^(R)
constexpr int kFacDecay = 3;  // 2^(G_last)
constexpr int kFacLast = 4;   // G_last          (exact mode)
constexpr int kFacOwn = 5;    // R_I             (exact mode)

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

// 16 per-key values of this lane's key set from an LDS row of 64.
__device__ __forceinline__ void lds_keys(const float *row, int kq, f32x8 out[2]) {
  out[0] = *reinterpret_cast<const f32x8 *>(row + kq);
  out[1] = *reinterpret_cast<const f32x8 *>(row + 32 + kq);
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

// Raw global loads for one chunk row of this lane (q, k, g) and 4*NVT values
// of one V row.
template <int NVT>
struct ChunkRegs {
  uint4 q[2], k[2];   // 2 x 8 keys of this lane's row (16-bit)
  float4 g[4];        // 16 log-gates (fp32 g) ...
  uint4 g16[2];       // ... or 16-bit g
  uint2 v[NVT];       // 4*NVT values of one V-tile row
};

template <bool GF32, int NVT>
__device__ __forceinline__ void load_chunk(ChunkRegs<NVT> &R, const uint16_t *__restrict__ q,
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
  const uint16_t *vp = v + (t_vrow * H + h) * V + vcol;
#pragma unroll
  for (int p = 0; p < NVT; ++p)
    R.v[p] = vrow_ok ? *reinterpret_cast<const uint2 *>(vp + 4 * p) : make_uint2(0, 0);
}

// Unpack 16 gates (log2 units) of this lane.
template <int DT, bool GF32, class R_>
__device__ __forceinline__ void unpack_gates(const R_ &R, f32x8 (&gs)[2]) {
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

// Split an fp32 state tile (4 values) into 16-bit high/low parts and store
// them transposed into the S^T buffers.
template <int DT, class SM>
__device__ __forceinline__ void store_state(SM &sm, int vcolumn, int krow, const f32x4 &S) {
  typedef Mfma<DT> M;
  const f32x8 s8 = {S[0], S[1], S[2], S[3], 0.f, 0.f, 0.f, 0.f};
  const typename M::Vec hi = M::cvt(s8);
  const typename M::Vec lo = M::cvt(s8 - M::widen(hi));
  const uint4 hb = to_bits(hi), lb = to_bits(lo);
  *reinterpret_cast<uint2 *>(&sm.sth[vcolumn][krow]) = make_uint2(hb.x, hb.y);
  *reinterpret_cast<uint2 *>(&sm.stl[vcolumn][krow]) = make_uint2(lb.x, lb.y);
}

struct ChunkArgs {
  const uint16_t *q, *k, *v;
  const void *g;
  const float *h0;
  uint16_t *o;
  float *ht;
  float *ws_state;   // [n_seq, H, P, K, V] fp32 (P > 1)
  float *ws_decay;   // [n_seq, H, P, K] fp32, log2 units (P > 1)
  int64_t bos;       // first row of the sequence
  int64_t len;       // rows of the sequence
  int c_beg, c_end;  // chunk range of the segment
  int H, V, h, n, v0, seg, P;
  float scale;
};

// Chunk range of segment `seg` of a sequence with `nch` chunks cut in P parts.
__device__ __forceinline__ void segment_range(int nch, int P, int seg, int &c0, int &c1) {
  const int per = (nch + P - 1) / P;
  c0 = min(seg * per, nch);
  c1 = min(c0 + per, nch);
}

// Entering state of segment seg >= 1 from the state-pass slots of its
// (sequence, head): slot 0 is the state after segment 0 (started from h0),
// slot s >= 1 the state segment s reaches from zero, with total log2 decay
// D(s):  S_e(1) = slot 0,  S_e(s+1) = 2^D(s) S_e(s) + slot s.
template <int NVT>
__device__ __forceinline__ void fold_entering_state(f32x4 (&S)[NVT], const float *__restrict__ ws_state,
                                                    const float *__restrict__ ws_decay, int64_t slot0,
                                                    int seg, int krow, int r, int V, int v0) {
#pragma unroll
  for (int t = 0; t < NVT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) S[t][i] = ws_state[(slot0 * KD + krow + i) * V + v0 + 16 * t + r];
  for (int s = 1; s < seg; ++s) {
    const float *src = ws_state + (slot0 + s) * KD * V;
    f32x4 d;
#pragma unroll
    for (int i = 0; i < 4; ++i) d[i] = fast_exp2(ws_decay[(slot0 + s) * KD + krow + i]);
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        S[t][i] = fmaf(d[i], S[t][i], src[static_cast<int64_t>(krow + i) * V + v0 + 16 * t + r]);
  }
}

// Kernel A body.  Wavefront wv (uniform) owns rows 16wv..16wv+15 of every
// chunk of the segment; the four wavefronts meet at two barriers per chunk.
template <int DT, bool GF32, int NVT>
__device__ __forceinline__ void segment_loop(SmemA<NVT> &sm, const ChunkArgs &a, const int wv, int lane) {
  typedef Mfma<DT> M;
  typedef typename M::Vec MV;
  const int r = lane & 15;        // row within block / MFMA column index
  const int gq = lane >> 4;       // lane group
  const int kq = 8 * gq;          // key offset of this lane inside each K=32 half
  const int H = a.H, V = a.V, h = a.h, v0 = a.v0;
  const int64_t len = a.len;

  // ---- entering state: rows 16wv + 4gq + i, columns v0 + 16t + r ----------
  const int64_t sbase = (static_cast<int64_t>(a.n) * H + h) * KD;
  const int krow = 16 * wv + 4 * gq;
  f32x4 S[NVT];
  if (a.seg == 0) {
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[t][i] = a.h0 ? a.h0[(sbase + krow + i) * V + v0 + 16 * t + r] : 0.f;
  } else {
    fold_entering_state<NVT>(S, a.ws_state, a.ws_decay, (static_cast<int64_t>(a.n) * H + h) * a.P, a.seg,
                             krow, r, V, v0);
  }
#pragma unroll
  for (int t = 0; t < NVT; ++t) store_state<DT>(sm, 16 * t + r, krow, S[t]);

  // V rows staged by this lane: row 16wv + lane/4, columns (lane%4)*4*NVT ..
  const int vrow = 16 * wv + (lane >> 2);
  const int vcl = (lane & 3) * 4 * NVT;
  const int vcol = v0 + vcl;
  const int row = 16 * wv + r;

  ChunkRegs<NVT> buf[2];
  if (a.c_beg < a.c_end) {
    const int64_t rem0 = len - static_cast<int64_t>(a.c_beg) * BT;
    const int64_t tb = a.bos + static_cast<int64_t>(a.c_beg) * BT;
    load_chunk<GF32, NVT>(buf[0], a.q, a.k, a.v, a.g, tb + row, row < rem0, tb + vrow, vrow < rem0, H, V,
                          h, kq, vcol);
  }

  for (int c2 = a.c_beg; c2 < a.c_end; c2 += 2) {
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int c = c2 + par;
    if (c >= a.c_end) break;
    const int64_t t0 = a.bos + static_cast<int64_t>(c) * BT;
    const int64_t rem = len - static_cast<int64_t>(c) * BT;   // valid rows in this chunk (>0)

    // ---- unpack: element e of half jj is key 32*jj + kq + e ---------------
    // The current buffer is consumed before the next prefetch is issued, so
    // the wait for it (at the loop head the compiler waits for every
    // outstanding load) never covers the prefetch.
    f32x8 qf[2], kf[2], gs[2];
    uint2 vv[NVT];
    {
      const ChunkRegs<NVT> &R = buf[par];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        qf[jj] = M::widen(from_bits<MV>(R.q[jj]));
        kf[jj] = M::widen(from_bits<MV>(R.k[jj]));
      }
      unpack_gates<DT, GF32>(R, gs);
#pragma unroll
      for (int p = 0; p < NVT; ++p) vv[p] = R.v[p];
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < a.c_end) {
      const int64_t rem2 = rem - BT;
      load_chunk<GF32, NVT>(buf[par ^ 1], a.q, a.k, a.v, a.g, t0 + BT + row, row < rem2, t0 + BT + vrow,
                            vrow < rem2, H, V, h, kq, vcol);
    }
    float gmax = fmaxf(gs[0][0], gs[1][0]);
#pragma unroll
    for (int e = 1; e < 8; ++e) gmax = fmaxf(gmax, fmaxf(gs[0][e], gs[1][e]));
    // ---- block-local inclusive cumsum over the 16 rows (DPP row scan) ------
    row_scan16(gs);
    if (r == 15) {
      *reinterpret_cast<f32x8 *>(&sm.tot[wv][kq]) = gs[0];
      *reinterpret_cast<f32x8 *>(&sm.tot[wv][32 + kq]) = gs[1];
    }
    const bool wpos = __builtin_amdgcn_ballot_w64(gmax > 0.f) != 0;
    if (lane == 0) sm.flag[wv] = wpos ? 1 : 0;
    lds_barrier();  // --------------------------------------------- barrier 1

    // ---- per-key references and factors (lane = key) -----------------------
    bool exact;
    {
      const int kk = lane;
      const float t0_ = sm.tot[0][kk], t1_ = sm.tot[1][kk], t2_ = sm.tot[2][kk], t3_ = sm.tot[3][kk];
      const float R1 = t0_, R2 = t0_ + t1_, R3 = R2 + t2_, GL = R3 + t3_;
      const float own = wv == 0 ? 0.f : wv == 1 ? R1 : wv == 2 ? R2 : R3;
      // without positive gates G2 falls monotonically, so |G2 - R| is largest
      // at the chunk ends: R (first half) and R - G_last (second half).
      const bool far = fmaxf(-R2, R2 - GL) > kRangeLimit;
      exact = (sm.flag[0] | sm.flag[1] | sm.flag[2] | sm.flag[3]) != 0 ||
              __builtin_amdgcn_ballot_w64(far) != 0;
      sm.fac[wv][kFacRel][kk] = own - R2;
      sm.fac[wv][kFacKs][kk] = fast_exp2(GL - R2);
      sm.fac[wv][kFacQ0][kk] = fast_exp2(R2);
      sm.fac[wv][kFacDecay][kk] = fast_exp2(GL);
      sm.fac[wv][kFacLast][kk] = GL;
      sm.fac[wv][kFacOwn][kk] = own;
    }
    // the state entering this chunk (computed at the end of the previous one);
    // every reader of the previous state passed barrier 1 already
    if (c > a.c_beg) {
#pragma unroll
      for (int t = 0; t < NVT; ++t) store_state<DT>(sm, 16 * t + r, krow, S[t]);
    }
    wave_sync_lds();
    // own-row decays of the state rows 16wv + 4gq + i
    const f32x4 sdec = *reinterpret_cast<const f32x4 *>(&sm.fac[wv][kFacDecay][krow]);

    // ---- operands ------------------------------------------------------------
    // fast: q~ = q 2^(G2 - R) (MFMA B operand of A^T), q~0 = q~ 2^R (of o_inter),
    //       k~ = k 2^(R - G2) (to LDS), k~s = k~ 2^(G_last - R) (to LDS, transposed)
    QK::Vec qtb[2];    // q~ as bf16 (fast) / q 2^(G2 - R_I) (exact, off-diagonal blocks)
    MV q0b[2];         // q~0 in the input dtype
    {
      f32x8 ks[2];
      if (!exact) {
        f32x8 rel[2], fks[2], fq0[2];
        lds_keys(sm.fac[wv][kFacRel], kq, rel);
        lds_keys(sm.fac[wv][kFacKs], kq, fks);
        lds_keys(sm.fac[wv][kFacQ0], kq, fq0);
        f32x8 kt[2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const f32x8 x = gs[jj] + rel[jj];             // G2 - R
          f32x8 eq, ek;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            eq[e] = fast_exp2(x[e]);
            ek[e] = fast_exp2(-x[e]);
          }
          const f32x8 qt = qf[jj] * eq;
          kt[jj] = kf[jj] * ek;
          ks[jj] = kt[jj] * fks[jj];
          qtb[jj] = QK::cvt(qt);
          q0b[jj] = M::cvt(qt * fq0[jj]);
        }
        *reinterpret_cast<uint4 *>(&sm.kt[row][kq]) = to_bits(QK::cvt(kt[0]));
        *reinterpret_cast<uint4 *>(&sm.kt[row][32 + kq]) = to_bits(QK::cvt(kt[1]));
      } else {
        f32x8 own8[2], gl[2];
        lds_keys(sm.fac[wv][kFacOwn], kq, own8);
        lds_keys(sm.fac[wv][kFacLast], kq, gl);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const f32x8 gabs = gs[jj] + own8[jj];
          f32x8 eq, e0, ek;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            eq[e] = fast_exp2(gs[jj][e]);                 // 2^(G2_i - R_I)
            e0[e] = fast_exp2(gabs[e]);                   // 2^(G2_i)
            ek[e] = fast_exp2(gl[jj][e] - gabs[e]);       // 2^(G_last - G2_j)
          }
          qtb[jj] = QK::cvt(qf[jj] * eq);
          q0b[jj] = M::cvt(qf[jj] * e0);
          ks[jj] = kf[jj] * ek;
          *reinterpret_cast<uint4 *>(&sm.xq[row][32 * jj + kq]) = to_bits(M::cvt(qf[jj]));
          *reinterpret_cast<uint4 *>(&sm.kt[row][32 * jj + kq]) = to_bits(M::cvt(kf[jj]));
          *reinterpret_cast<f32x8 *>(&sm.xg[row][32 * jj + kq]) = gabs;
        }
      }
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const uint4 kb = to_bits(M::cvt(ks[jj]));
        const uint32_t w4[4] = {kb.x, kb.y, kb.z, kb.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          sm.kst[32 * jj + kq + e][row] =
              static_cast<uint16_t>((e & 1) ? (w4[e >> 1] >> 16) : (w4[e >> 1] & 0xffffu));
      }
    }
#pragma unroll
    for (int p = 0; p < NVT; ++p) {
      sm.vt[vcl + 4 * p + 0][vrow] = static_cast<uint16_t>(vv[p].x & 0xffffu);
      sm.vt[vcl + 4 * p + 1][vrow] = static_cast<uint16_t>(vv[p].x >> 16);
      sm.vt[vcl + 4 * p + 2][vrow] = static_cast<uint16_t>(vv[p].y & 0xffffu);
      sm.vt[vcl + 4 * p + 3][vrow] = static_cast<uint16_t>(vv[p].y >> 16);
    }
    lds_barrier();  // --------------------------------------------- barrier 2

    // ---- A^T blocks (rows j of block J, columns i of this block) ------------
    // blocks J > wv are zero, block J == wv is causally masked.
    f32x4 at[4];
    if (!exact) {
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        at[J] = (f32x4){0.f, 0.f, 0.f, 0.f};
        if (J <= wv) {
          const QK::Vec a0 = from_bits<QK::Vec>(*reinterpret_cast<const uint4 *>(&sm.kt[16 * J + r][kq]));
          const QK::Vec a1 = from_bits<QK::Vec>(*reinterpret_cast<const uint4 *>(&sm.kt[16 * J + r][32 + kq]));
          at[J] = QK::mma(a0, qtb[0], at[J]);
          at[J] = QK::mma(a1, qtb[1], at[J]);
        }
      }
    } else {
      f32x8 own8[2];
      lds_keys(sm.fac[wv][kFacOwn], kq, own8);
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        at[J] = (f32x4){0.f, 0.f, 0.f, 0.f};
        if (J < wv) {   // off-diagonal: k re-referenced to R_I (<= 1 for decays)
          const int jrow = 16 * J + r;
          QK::Vec kj[2];
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const f32x8 kr = M::widen(from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.kt[jrow][32 * jj + kq])));
            const f32x8 gr = *reinterpret_cast<const f32x8 *>(&sm.xg[jrow][32 * jj + kq]);
            f32x8 e2;
#pragma unroll
            for (int e = 0; e < 8; ++e) e2[e] = fast_exp2(own8[jj][e] - gr[e]);
            kj[jj] = QK::cvt(kr * e2);
          }
          at[J] = QK::mma(kj[0], qtb[0], at[J]);
          at[J] = QK::mma(kj[1], qtb[1], at[J]);
        }
      }
      // diagonal block elementwise: lane holds A[i = r][j = 4gq + ii]
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int j = 4 * gq + ii;
        const int jrow = 16 * wv + j;
        float acc = 0.f;
        if (j <= r) {
#pragma unroll 1
          for (int k8 = 0; k8 < KD; k8 += 8) {
            const f32x8 qv = M::widen(from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.xq[row][k8])));
            const f32x8 kv = M::widen(from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.kt[jrow][k8])));
            const f32x8 gi = *reinterpret_cast<const f32x8 *>(&sm.xg[row][k8]);
            const f32x8 gj = *reinterpret_cast<const f32x8 *>(&sm.xg[jrow][k8]);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += qv[e] * kv[e] * fast_exp2(gi[e] - gj[e]);
          }
        }
#pragma unroll
        for (int J = 0; J < 4; ++J)
          if (J == wv) at[J][ii] = acc;
      }
    }
    // causal mask on the diagonal block (row i = r, column j = 4gq + ii)
#pragma unroll
    for (int J = 0; J < 4; ++J)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        if (J == wv && 4 * gq + ii > r) at[J][ii] = 0.f;
    // A as the B operand of V^T A^T: K slots 0-3 <- block 2pr, 4-7 <- block 2pr+1
    MV ab[2];
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      const f32x8 av = {at[2 * pr][0], at[2 * pr][1], at[2 * pr][2], at[2 * pr][3],
                        at[2 * pr + 1][0], at[2 * pr + 1][1], at[2 * pr + 1][2], at[2 * pr + 1][3]};
      ab[pr] = M::cvt(av);
    }

    // ---- per V tile: o^T = S^T q~0^T + V^T A^T, store, state update ----------
#pragma unroll
    for (int t = 0; t < NVT; ++t) {
      const int vc = 16 * t + r;
      f32x4 oacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const MV shi = from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.sth[vc][32 * jj + kq]));
        const MV slo = from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.stl[vc][32 * jj + kq]));
        oacc = M::mma(shi, q0b[jj], oacc);
        oacc = M::mma(slo, q0b[jj], oacc);
      }
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        if (2 * pr <= wv) {
          const uint2 va = *reinterpret_cast<const uint2 *>(&sm.vt[vc][32 * pr + 4 * gq]);
          const uint2 vb = *reinterpret_cast<const uint2 *>(&sm.vt[vc][32 * pr + 16 + 4 * gq]);
          oacc = M::mma(from_bits<MV>(make_uint4(va.x, va.y, vb.x, vb.y)), ab[pr], oacc);
        }
      }
      if (row < rem) {
        const f32x8 o8 = {oacc[0] * a.scale, oacc[1] * a.scale, oacc[2] * a.scale, oacc[3] * a.scale,
                          0.f, 0.f, 0.f, 0.f};
        const uint4 ob = to_bits(M::cvt(o8));
        *reinterpret_cast<uint2 *>(a.o + ((t0 + row) * H + h) * V + v0 + 16 * t + 4 * gq) =
            make_uint2(ob.x, ob.y);
      }
      // S <- 2^(G_last) S + Ks^T V for the state rows of this wavefront
      S[t] *= sdec;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const MV ka = from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.kst[row][32 * jj + kq]));
        const MV vb = from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.vt[vc][32 * jj + kq]));
        S[t] = M::mma(ka, vb, S[t]);
      }
    }
  }
  }

  // ---- final state of the sequence -----------------------------------------
  if (a.seg == a.P - 1 && a.ht) {
#pragma unroll
    for (int t = 0; t < NVT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) a.ht[(sbase + krow + i) * V + v0 + 16 * t + r] = S[t][i];
  }
}

template <int DT, bool GF32, int NVT>
__global__ __launch_bounds__(256, 2) void gla_chunk_segment_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, const void *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int64_t T, int H, int V, float scale,
    const float *__restrict__ h0, uint16_t *__restrict__ o, float *__restrict__ ht, int P,
    float *__restrict__ ws_state, float *__restrict__ ws_decay) {
  __shared__ SmemA<NVT> sm;
  const int nvg = V / (16 * NVT);
  // block -> (sequence, head, V group, segment); the segments of one
  // (sequence, head) are consecutive
  int64_t b = blockIdx.x;
  ChunkArgs a;
  a.P = P;
  a.seg = static_cast<int>(b % P);
  b /= P;
  const int vg = static_cast<int>(b % nvg);
  b /= nvg;
  a.h = static_cast<int>(b % H);
  a.n = static_cast<int>(b / H);
  a.q = q; a.k = k; a.v = v; a.g = g; a.h0 = h0; a.o = o; a.ht = ht;
  a.ws_state = ws_state; a.ws_decay = ws_decay;
  a.H = H; a.V = V; a.scale = scale;
  a.v0 = vg * 16 * NVT;
  a.bos = min(max(cu_seqlens[a.n], (int64_t)0), T);
  const int64_t eos = min(max(cu_seqlens[a.n + 1], a.bos), T);
  a.len = eos - a.bos;
  segment_range(static_cast<int>((a.len + BT - 1) / BT), P, a.seg, a.c_beg, a.c_end);
  segment_loop<DT, GF32, NVT>(sm, a, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), threadIdx.x & 63);
}

// ------------------------------------------------------------ kernel S ----
template <int NVT>
struct __align__(16) SmemS {
  uint16_t kst[KD][kTP];         // k~s transposed (key k, row j), input dtype
  uint16_t vt[16 * NVT][kTP];    // V tile transposed (column v, row j)
  float tot[2][4][KD];           // per-block column sums of g, by chunk parity
};

// State-only walk over segment seg (< P - 1) of one (sequence, head, V
// group):  S <- 2^(G_last) S + (k 2^(G_last - G))^T v  per chunk, from h0
// for segment 0 and from zero otherwise.  Writes the workspace slot and,
// for seg >= 1, the segment's total log2 decay.
template <int DT, bool GF32, int NVT>
__global__ __launch_bounds__(256, 2) void gla_chunk_state_kernel(
    const uint16_t *__restrict__ k, const uint16_t *__restrict__ v, const void *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int64_t T, int H, int V,
    const float *__restrict__ h0, int P, float *__restrict__ ws_state, float *__restrict__ ws_decay) {
  typedef Mfma<DT> M;
  typedef typename M::Vec MV;
  __shared__ SmemS<NVT> sm;
  const int nvg = V / (16 * NVT);
  int64_t b = blockIdx.x;
  const int seg = static_cast<int>(b % (P - 1));
  b /= (P - 1);
  const int vg = static_cast<int>(b % nvg);
  b /= nvg;
  const int h = static_cast<int>(b % H);
  const int n = static_cast<int>(b / H);
  const int v0 = vg * 16 * NVT;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, gq = lane >> 4, kq = 8 * gq;
  const int krow = 16 * wv + 4 * gq;
  const int row = 16 * wv + r;
  const int vrow = 16 * wv + (lane >> 2);
  const int vcl = (lane & 3) * 4 * NVT;

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

  struct StateRegs {
    uint4 k[2];
    float4 g[4];
    uint4 g16[2];
    uint2 v[NVT];
  };
  auto load_state = [&](StateRegs &R, int c) {
    const int64_t t0 = bos + static_cast<int64_t>(c) * BT;
    const int64_t rem = len - static_cast<int64_t>(c) * BT;
    const bool ok = row < rem;
    const int64_t base = ((t0 + row) * H + h) * KD;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      R.k[jj] = ok ? *reinterpret_cast<const uint4 *>(k + base + 32 * jj + kq) : make_uint4(0, 0, 0, 0);
      if (GF32) {
        const float *gp = static_cast<const float *>(g) + base + 32 * jj + kq;
        R.g[2 * jj] = ok ? *reinterpret_cast<const float4 *>(gp) : make_float4(0.f, 0.f, 0.f, 0.f);
        R.g[2 * jj + 1] = ok ? *reinterpret_cast<const float4 *>(gp + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        R.g16[jj] = ok ? *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(g) + base + 32 * jj + kq)
                       : make_uint4(0, 0, 0, 0);
      }
    }
    const bool vok = vrow < rem;
    const uint16_t *vp = v + ((t0 + vrow) * H + h) * V + v0 + vcl;
#pragma unroll
    for (int p = 0; p < NVT; ++p)
      R.v[p] = vok ? *reinterpret_cast<const uint2 *>(vp + 4 * p) : make_uint2(0, 0);
  };

  StateRegs sb[2];
  if (c_beg < c_end) load_state(sb[0], c_beg);
  for (int c2 = c_beg; c2 < c_end; c2 += 2) {
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int c = c2 + par;
    if (c >= c_end) break;
    f32x8 kf[2], gs[2];
    uint2 vv[NVT];
    {
      const StateRegs &R = sb[par];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) kf[jj] = M::widen(from_bits<MV>(R.k[jj]));
      unpack_gates<DT, GF32>(R, gs);
#pragma unroll
      for (int p = 0; p < NVT; ++p) vv[p] = R.v[p];
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < c_end) load_state(sb[par ^ 1], c + 1);
    row_scan16(gs);
    if (r == 15) {
      *reinterpret_cast<f32x8 *>(&sm.tot[par][wv][kq]) = gs[0];
      *reinterpret_cast<f32x8 *>(&sm.tot[par][wv][32 + kq]) = gs[1];
    }
    lds_barrier();  // ------------------------------ barrier 1 (totals ready)
    // G_abs - G_last for this lane's keys; state decay of its rows
    f32x8 off[2], gl[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      off[jj] = (f32x8){0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      gl[jj] = off[jj];
    }
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      f32x8 tj[2];
      lds_keys(sm.tot[par][J], kq, tj);
      if (J < wv) {
        off[0] += tj[0];
        off[1] += tj[1];
      }
      gl[0] += tj[0];
      gl[1] += tj[1];
    }
    f32x4 sdec;
    {
      float d4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        const f32x4 tj = *reinterpret_cast<const f32x4 *>(&sm.tot[par][J][krow]);
#pragma unroll
        for (int i = 0; i < 4; ++i) d4[i] += tj[i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) sdec[i] = fast_exp2(d4[i]);
      if (wv == 0 && seg > 0) {
        float dl = 0.f;
#pragma unroll
        for (int J = 0; J < 4; ++J) dl += sm.tot[par][J][lane];
        dsum += dl;
      }
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      f32x8 e2;
#pragma unroll
      for (int e = 0; e < 8; ++e) e2[e] = fast_exp2(gl[jj][e] - (gs[jj][e] + off[jj][e]));
      const uint4 kb = to_bits(M::cvt(kf[jj] * e2));
      const uint32_t w4[4] = {kb.x, kb.y, kb.z, kb.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        sm.kst[32 * jj + kq + e][row] =
            static_cast<uint16_t>((e & 1) ? (w4[e >> 1] >> 16) : (w4[e >> 1] & 0xffffu));
    }
#pragma unroll
    for (int p = 0; p < NVT; ++p) {
      sm.vt[vcl + 4 * p + 0][vrow] = static_cast<uint16_t>(vv[p].x & 0xffffu);
      sm.vt[vcl + 4 * p + 1][vrow] = static_cast<uint16_t>(vv[p].x >> 16);
      sm.vt[vcl + 4 * p + 2][vrow] = static_cast<uint16_t>(vv[p].y & 0xffffu);
      sm.vt[vcl + 4 * p + 3][vrow] = static_cast<uint16_t>(vv[p].y >> 16);
    }
    lds_barrier();  // ------------------------------ barrier 2 (k~s, V ready)
#pragma unroll
    for (int t = 0; t < NVT; ++t) {
      S[t] *= sdec;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const MV ka = from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.kst[row][32 * jj + kq]));
        const MV vb = from_bits<MV>(*reinterpret_cast<const uint4 *>(&sm.vt[16 * t + r][32 * jj + kq]));
        S[t] = M::mma(ka, vb, S[t]);
      }
    }
    // kst / vt are rewritten after the next chunk's barrier 1, which every
    // wavefront reaches only after these reads
  }
  }

  const int64_t slot = (static_cast<int64_t>(n) * H + h) * P + seg;
  float *dst = ws_state + slot * KD * V;
#pragma unroll
  for (int t = 0; t < NVT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[static_cast<int64_t>(krow + i) * V + v0 + 16 * t + r] = S[t][i];
  if (wv == 0 && v0 == 0) ws_decay[slot * KD + lane] = dsum;
}

inline int pick_nvt(int V) {
  const int tiles = V / 16;
  for (int nvt = 4; nvt >= 1; --nvt)
    if (tiles % nvt == 0) return nvt;
  return 1;
}

// Segments per sequence: about two workgroups per CU (256 CUs), at least two
// chunks per segment on average, at most 64 segments.
inline int pick_segments(int n_seq, int64_t T, int H, int V) {
  const int nvg = V / (16 * pick_nvt(V));
  const int64_t chains = static_cast<int64_t>(n_seq) * H * nvg;
  if (chains <= 0) return 1;
  int64_t p = (512 + chains - 1) / chains;
  const int64_t avg_chunks = (T / std::max<int64_t>(n_seq, 1) + BT - 1) / BT;
  p = std::min<int64_t>(p, std::max<int64_t>(1, avg_chunks / 2));
  p = std::min<int64_t>(p, 64);
  return static_cast<int>(std::max<int64_t>(p, 1));
}

inline size_t workspace_bytes_for(int n_seq, int H, int V, int P) {
  if (P <= 1) return 0;
  const size_t slots = static_cast<size_t>(n_seq) * H * P;
  return slots * KD * V * sizeof(float) + slots * KD * sizeof(float);
}

template <int DT, bool GF32, int NVT>
int launch_nvt(const void *q, const void *k, const void *v, const void *g, const int64_t *cu, int n_seq,
               int64_t T, int H, int V, float scale, const float *h0, void *o, float *ht, int P,
               float *ws_state, float *ws_decay, hipStream_t st) {
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
                       g, cu, n_seq, T, H, V, h0, P, ws_state, ws_decay);
  }
  hipLaunchKernelGGL((gla_chunk_segment_kernel<DT, GF32, NVT>), dim3(static_cast<unsigned>(blocks_a)),
                     dim3(256), 0, st, q16, static_cast<const uint16_t *>(k),
                     static_cast<const uint16_t *>(v), g, cu, n_seq, T, H, V, scale, h0, o16, ht, P,
                     ws_state, ws_decay);
  return launch_status("gla_chunk_fwd");
}

template <int DT, bool GF32>
int launch_chunk(const void *q, const void *k, const void *v, const void *g, const int64_t *cu, int n_seq,
                 int64_t T, int H, int V, float scale, const float *h0, void *o, float *ht, int P,
                 float *ws_state, float *ws_decay, hipStream_t st) {
  switch (pick_nvt(V)) {
    case 4: return launch_nvt<DT, GF32, 4>(q, k, v, g, cu, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_decay, st);
    case 3: return launch_nvt<DT, GF32, 3>(q, k, v, g, cu, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_decay, st);
    case 2: return launch_nvt<DT, GF32, 2>(q, k, v, g, cu, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_decay, st);
    default: return launch_nvt<DT, GF32, 1>(q, k, v, g, cu, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_decay, st);
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
  const int P = pick_segments(n_seq, T, H, V);
  const size_t need = workspace_bytes_for(n_seq, H, V, P);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("gla_chunk_fwd: workspace of %zu bytes needed (ssla_gla_chunk_workspace_size), %zu given",
              need, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(need == 0 || aligned(workspace, 16), "gla_chunk_fwd: workspace must be 16-byte aligned");
  float *ws_state = static_cast<float *>(workspace);
  float *ws_decay = need ? ws_state + static_cast<size_t>(n_seq) * H * P * KD * V : nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool gf32 = g_dtype == SSLA_F32;
  if (dtype == SSLA_BF16)
    return gf32 ? launch_chunk<SSLA_BF16, true>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_decay, st)
                : launch_chunk<SSLA_BF16, false>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_decay, st);
  return gf32 ? launch_chunk<SSLA_F16, true>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_decay, st)
              : launch_chunk<SSLA_F16, false>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, o, ht, P, ws_state, ws_decay, st);
}
