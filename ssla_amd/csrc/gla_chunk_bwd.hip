// Chunked gated-linear-attention backward on gfx950.
//
// Gradients of the forward in gla_chunk.hip (reference ChunkGLAFunction.
// backward / chunk_gla_bwd, ops/gla/chunk.py:963-1053, 1096-1116): given do
// (and dht, the gradient of the final state), dq, dk, dv, dg and dh0.
//
// Math, per sequence and head, chunks of 64 rows, G = chunk-local inclusive
// cumsum of g, h[c] = state entering chunk c, dh[c] = gradient of the state
// leaving chunk c (from the chunks after it and dht):
//   dA_ts = scale do_t . v_s                               (s <= t)
//   A_ts  = scale sum_k q_tk k_sk e^(G_tk - G_sk)          (s <= t)
//   dq_t  = sum_s dA_ts e^(G_t - G_s) k_s + scale e^(G_t) (h[c] do_t)
//   dk_s  = sum_t dA_ts e^(G_t - G_s) q_t + e^(G_last - G_s) (dh[c] v_s)
//   dv_s  = sum_t A_ts do_t + (k_s e^(G_last - G_s))^T dh[c]
//   dg_t  = sum_{s >= t in the chunk} (q dq - k dk)_s + sum_v dh[c] h[c+1]
// The last line is the reverse cumsum over the whole sequence of
// q dq - k dk plus the dht . ht term: the part after chunk c equals
// sum_v dh[c] * (state leaving chunk c), which needs no cross-chunk pass.
//   h[c+1]  = e^(G_last) h[c] + (k e^(G_last - G))^T v        (forward)
//   dh[c-1] = e^(G_last) dh[c] + (scale q e^(G))^T do         (reverse)
// with h[0] = h0 (or 0), dh[last] = dht (or 0) and dh0 = dh[-1].
//
// Launches: offsets (chunk and state-slot offsets per sequence), the
// forward state pass and the reverse state pass (one wavefront per
// (sequence, head, 16 value columns), serial over chunks, writing every
// chunk's entering state / leaving-state gradient to workspace slots), and
// the chunk kernel (one workgroup per (chunk, head), fully parallel).
//
// Exponents are in log2 units and every factor is referenced to a point
// inside the span it covers (as in the forward): with E_I = G at the last row
// of 16-row block I (E_-1 = 0) and M_I = (E_I-1 + E_I) / 2, rows t of block I
// use e^(G_t - M_I) on the output side and e^(M_I - G_s) on the operand side,
// so for non-positive gates no factor exceeds the decay over half a block.
// Exponents are clamped to +-126.  Products run on v_mfma_f32_16x16x32_bf16
// as split bf16 products (see mmax) with fp32 accumulation; states, A, dA
// and dg are fp32.
#include "common.h"

namespace ssla {
namespace {

constexpr int BT = 64;   // chunk rows
constexpr int KD = 64;   // key width
constexpr float kClamp = 126.f;

__device__ __forceinline__ float cexp2(float x) { return fast_exp2(fminf(fmaxf(x, -kClamp), kClamp)); }

// a . b for fp32 operands as three bf16 products (hi hi + hi lo + lo hi, each
// operand split into a bf16 head and the bf16 of its remainder): about 16
// mantissa bits per operand.  dg is a reverse cumsum of q dq - k dk, whose
// terms cancel (strongly so for fast-decaying gates); single bf16 operands
// leave it with errors of several percent.
// AX / BX: the operand is an exact bf16 value (a bf16 input), so its
// remainder is zero and its lo product is skipped.
typedef float f32x8 __attribute__((ext_vector_type(8)));
template <bool AX, bool BX>
__device__ __forceinline__ f32x4 mmax(const float (&a)[8], const float (&b)[8], f32x4 c) {
  const f32x8 va = {a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7]};
  const f32x8 vb = {b[0], b[1], b[2], b[3], b[4], b[5], b[6], b[7]};
  const bf16x8 ah = __builtin_convertvector(va, bf16x8), bh = __builtin_convertvector(vb, bf16x8);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
  if constexpr (!BX) {
    const bf16x8 bl = __builtin_convertvector(vb - __builtin_convertvector(bh, f32x8), bf16x8);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
  }
  if constexpr (!AX) {
    const bf16x8 al = __builtin_convertvector(va - __builtin_convertvector(ah, f32x8), bf16x8);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
  }
  return c;
}

// 16-bit input element <-> fp32
template <int DT> struct Elt;
template <> struct Elt<SSLA_BF16> {
  static __device__ __forceinline__ float f(uint16_t b) { return bf16_bits_to_f32(b); }
  static __device__ __forceinline__ uint16_t b(float x) { return f32_to_bf16_bits(x); }
};
template <> struct Elt<SSLA_F16> {
  static __device__ __forceinline__ float f(uint16_t b) { return static_cast<float>(__builtin_bit_cast(_Float16, b)); }
  static __device__ __forceinline__ uint16_t b(float x) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x)); }
};

template <bool GF32, int DT>
__device__ __forceinline__ float load_g(const void *g, int64_t i) {
  if constexpr (GF32) return static_cast<const float *>(g)[i];
  else return Elt<DT>::f(static_cast<const uint16_t *>(g)[i]);
}

__device__ __forceinline__ void seq_bounds(const int64_t *cu, int n, int64_t T, int64_t &bos, int64_t &eos) {
  bos = min(max(cu[n], (int64_t)0), T);
  eos = min(max(cu[n + 1], bos), T);
}

// Chunks per segment of the state passes.  At C2 (4096 chunk-heads) 16
// measured the same state-pass time as 8 with half the fold work
// (fold 7.9 vs 12.8 us); 4 was slower.
constexpr int kSegC = 16;

// coff[n] = chunks of sequences 0..n-1 and sgoff[n] = their segments of
// kSegC chunks (coff[n_seq], sgoff[n_seq]: the totals).  One workgroup.
__global__ __launch_bounds__(256) void bwd_offsets_kernel(const int64_t *__restrict__ cu, int n_seq, int64_t T,
                                                          int64_t *__restrict__ coff, int64_t *__restrict__ sgoff) {
  __shared__ int64_t pc[256], ps[256];
  int64_t carry_c = 0, carry_s = 0;
  for (int base = 0; base < n_seq; base += 256) {
    const int n = base + static_cast<int>(threadIdx.x);
    int64_t c = 0;
    if (n < n_seq) {
      int64_t bos, eos;
      seq_bounds(cu, n, T, bos, eos);
      c = (eos - bos + BT - 1) / BT;
    }
    const int64_t sgc = (c + kSegC - 1) / kSegC;
    pc[threadIdx.x] = c;
    ps[threadIdx.x] = sgc;
    __syncthreads();
    for (int d = 1; d < 256; d <<= 1) {   // inclusive scans (Hillis-Steele)
      const bool up = threadIdx.x >= static_cast<unsigned>(d);
      const int64_t xc = up ? pc[threadIdx.x - d] : 0, xs = up ? ps[threadIdx.x - d] : 0;
      __syncthreads();
      pc[threadIdx.x] += xc;
      ps[threadIdx.x] += xs;
      __syncthreads();
    }
    if (n < n_seq) {
      coff[n] = carry_c + pc[threadIdx.x] - c;
      sgoff[n] = carry_s + ps[threadIdx.x] - sgc;
    }
    carry_c += pc[255];
    carry_s += ps[255];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    coff[n_seq] = carry_c;
    sgoff[n_seq] = carry_s;
  }
}

// --------------------------------------------------------- state passes --
// Each sequence's chunks are cut into segments of kSegC chunks.  A local
// pass runs every segment from a zero state (one workgroup per (segment,
// head); wavefront w owns value columns 16 w .. 16 w + 15, lane l holds
// keys 16 Kb + 4 (l / 16) + i of tile Kb, column l % 16):
// * forward (REV = false): X = k, Y = v, factor e^(G_last - G_t); stores the
//   local state entering each chunk, the log2 decay from the segment start
//   to it, and the segment's local end state and total decay;
// * reverse (REV = true): X = scale q, Y = do, factor e^(G_t), chunks in
//   reverse; stores the local gradient of the state entering each chunk and
//   the log2 decay from there to the segment end.
// The fold then carries states across segments, and the chunk kernel adds
// the carried part: state = local + 2^decay * carried (per key).
// All loads of a chunk are issued at once (16-byte pieces, every thread),
// and the next chunk's pieces are in flight while the current one runs.

struct __align__(16) SmemP {
  uint16_t x[BT][KD];
  float g[BT][KD];     // raw gates, then the log2 cumsum
  uint16_t y[BT][64];
  float glast[KD];
  float psum[4][KD];
};

// Finds n with off[n] <= i < off[n + 1] (the last n with off[n] <= i).
__device__ __forceinline__ int find_seq(const int64_t *off, int n_seq, int64_t i) {
  int lo = 0, hi = n_seq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (off[mid] <= i) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Log2 cumsum of the staged gates of one chunk (in place) by NT threads:
// NT / 64 threads per key, each over 64 / (NT / 64) consecutive rows.
template <int NT, int LD>
__device__ __forceinline__ void gate_cumsum(float (&gt)[BT][LD], float (&psum)[NT / 64][KD], float *glast) {
  constexpr int NQ = NT / 64, RQ = BT / NQ;
  const int key = threadIdx.x & 63, qd = threadIdx.x >> 6;
  float run[RQ];
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < RQ; ++r) {
    s += gt[RQ * qd + r][key];
    run[r] = s;
  }
  psum[qd][key] = s;
  __syncthreads();
  float off = 0.f;
  for (int b = 0; b < qd; ++b) off += psum[b][key];
#pragma unroll
  for (int r = 0; r < RQ; ++r) gt[RQ * qd + r][key] = (run[r] + off) * kLog2e;
  if (qd == NQ - 1) glast[key] = (s + off) * kLog2e;
  __syncthreads();
}

template <bool REV, int DT, bool GF32>
__device__ __forceinline__ void seg_pass(SmemP &sm, const int64_t bid, const uint16_t *__restrict__ X,
                                         const uint16_t *__restrict__ Y, const void *__restrict__ g,
                                         const int64_t *__restrict__ cu, const int64_t *__restrict__ coff,
                                         const int64_t *__restrict__ sgoff, int n_seq, int64_t T, int H, int V,
                                         float xscale, float *__restrict__ loc, float *__restrict__ dec,
                                         float *__restrict__ eloc, float *__restrict__ dtot) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int h = static_cast<int>(bid % H);
  const int64_t sg = bid / H;
  if (sg >= sgoff[n_seq]) return;   // workgroup-uniform
  const int n = find_seq(sgoff, n_seq, sg);
  int64_t bos, eos;
  seq_bounds(cu, n, T, bos, eos);
  const int64_t nc = (eos - bos + BT - 1) / BT;
  const int64_t j0 = (sg - sgoff[n]) * kSegC;   // first chunk of the segment in the sequence
  const int m = static_cast<int>(min(static_cast<int64_t>(kSegC), nc - j0));
  const int64_t c0 = coff[n] + j0;              // its global chunk index
  const int v0 = 16 * w;
  const bool active = v0 < V;
  const int64_t KV = static_cast<int64_t>(KD) * V;
  const int nyp = BT * V / 8;                   // 16-byte pieces of a chunk's Y rows

  // prefetch registers: X 2 pieces, g 4 (fp32) or 2 (16-bit), Y up to 2
  uint4 px[2], pg[4], py[2];
  auto fetch = [&](int64_t j) {
    const int64_t t0 = bos + j * BT;
    const int nrows = static_cast<int>(min(static_cast<int64_t>(BT), eos - t0));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid * 2 + i, r = e >> 3, pc = e & 7;
      px[i] = r < nrows ? *reinterpret_cast<const uint4 *>(X + ((t0 + r) * H + h) * KD + pc * 8) : uint4{0, 0, 0, 0};
    }
    if constexpr (GF32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = tid * 4 + i, r = e >> 4, pc = e & 15;
        pg[i] = r < nrows ? *reinterpret_cast<const uint4 *>(static_cast<const float *>(g) + ((t0 + r) * H + h) * KD + pc * 4)
                          : uint4{0, 0, 0, 0};
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid * 2 + i, r = e >> 3, pc = e & 7;
        pg[i] = r < nrows ? *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(g) + ((t0 + r) * H + h) * KD + pc * 8)
                          : uint4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 256 * i;
      const int r = e / (V / 8), pc = e % (V / 8);
      py[i] = (e < nyp && r < nrows) ? *reinterpret_cast<const uint4 *>(Y + ((t0 + r) * H + h) * V + pc * 8)
                                     : uint4{0, 0, 0, 0};
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid * 2 + i;
      *reinterpret_cast<uint4 *>(&sm.x[e >> 3][(e & 7) * 8]) = px[i];
    }
    if constexpr (GF32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = tid * 4 + i;
        *reinterpret_cast<uint4 *>(&sm.g[e >> 4][(e & 15) * 4]) = pg[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid * 2 + i, r = e >> 3, pc = e & 7;
        const uint16_t *u = reinterpret_cast<const uint16_t *>(&pg[i]);
#pragma unroll
        for (int q = 0; q < 8; ++q) sm.g[r][pc * 8 + q] = Elt<DT>::f(u[q]);
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 256 * i;
      if (e < nyp) *reinterpret_cast<uint4 *>(&sm.y[e / (V / 8)][(e % (V / 8)) * 8]) = py[i];
    }
  };

  f32x4 acc[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) acc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float D = 0.f;   // lane = key (wavefront 0): log2 decay accumulated so far
  auto store_loc = [&](int64_t c) {
    if (active) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          loc[(c * H + h) * KV + static_cast<int64_t>(kb * 16 + grp * 4 + i) * V + v0 + col] = acc[kb][i];
    }
    if (w == 0) dec[(c * H + h) * KD + lane] = D;
  };

  fetch(REV ? j0 + m - 1 : j0);
  for (int it = 0; it < m; ++it) {
    const int64_t j = REV ? j0 + m - 1 - it : j0 + it;
    stage();
    if (it + 1 < m) fetch(REV ? j - 1 : j + 1);   // next chunk in flight
    __syncthreads();
    gate_cumsum<256>(sm.g, sm.psum, sm.glast);
    if (!REV) store_loc(c0 + (j - j0));
    if (active) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[kb][i] *= cexp2(sm.glast[kb * 16 + grp * 4 + i]);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          float a[8], b[8];
          const int key = kb * 16 + col;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int t = ks * 32 + grp * 8 + e;
            const float x = Elt<DT>::f(sm.x[t][key]) * xscale;
            a[e] = x * cexp2(REV ? sm.g[t][key] : sm.glast[key] - sm.g[t][key]);
            b[e] = Elt<DT>::f(sm.y[t][v0 + col]);
          }
          acc[kb] = mmax<false, DT == SSLA_BF16>(a, b, acc[kb]);
        }
      }
    }
    D += sm.glast[lane];
    if (REV) store_loc(c0 + (j - j0));
    __syncthreads();   // the LDS tiles are rewritten by the next chunk
  }
  if (!REV) {
    if (active) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          eloc[(sg * H + h) * KV + static_cast<int64_t>(kb * 16 + grp * 4 + i) * V + v0 + col] = acc[kb][i];
    }
    if (w == 0) dtot[(sg * H + h) * KD + lane] = D;
  }
}

// Both passes in one launch: blocks [0, nb) run the forward pass (X = k,
// Y = v), blocks [nb, 2 nb) the reverse pass (X = scale q, Y = do); they are
// independent, so the two halves fill the GPU together.
template <int DT, bool GF32>
__global__ __launch_bounds__(256) void bwd_seg_passes(const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
                                                      const uint16_t *__restrict__ q, const uint16_t *__restrict__ dout,
                                                      const void *__restrict__ g, const int64_t *__restrict__ cu,
                                                      const int64_t *__restrict__ coff,
                                                      const int64_t *__restrict__ sgoff, int n_seq, int64_t T, int H,
                                                      int V, float scale, int64_t nb, float *__restrict__ hloc,
                                                      float *__restrict__ dfw, float *__restrict__ eloc,
                                                      float *__restrict__ dtot, float *__restrict__ dloc,
                                                      float *__restrict__ drv) {
  __shared__ SmemP sm;
  const int64_t b = blockIdx.x;
  if (b < nb)
    seg_pass<false, DT, GF32>(sm, b, k, v, g, cu, coff, sgoff, n_seq, T, H, V, 1.f, hloc, dfw, eloc, dtot);
  else
    seg_pass<true, DT, GF32>(sm, b - nb, q, dout, g, cu, coff, sgoff, n_seq, T, H, V, scale, dloc, drv, nullptr,
                             nullptr);
}

// Carries states across the segments of one (sequence, head):
//   Sin[0] = h0 (or 0), Sin[s+1] = 2^Dtot[s] Sin[s] + Eloc[s] (Sin[nseg] = ht)
//   dSend[nseg-1] = dht (or 0), dSend[s-1] = 2^Dtot[s] dSend[s] + dloc[first chunk of s]
// and dh0 = 2^Dtot[0] dSend[0] + dloc[first chunk].  Sin has nseg + 1
// entries per sequence (index sgoff[n] + n + s).
__global__ __launch_bounds__(256) void bwd_fold_kernel(const int64_t *__restrict__ coff,
                                                       const int64_t *__restrict__ sgoff, int n_seq, int H, int V,
                                                       const float *__restrict__ h0, const float *__restrict__ dht,
                                                       const float *__restrict__ eloc, const float *__restrict__ dtot,
                                                       const float *__restrict__ dloc, float *__restrict__ sin_,
                                                       float *__restrict__ dsend, float *__restrict__ dh0) {
  // one thread per (sequence, head, state element)
  const int64_t KV = static_cast<int64_t>(KD) * V;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t idx = gid % KV;
  const int h = static_cast<int>((gid / KV) % H);
  const int n = static_cast<int>(gid / (KV * H));
  if (n >= n_seq) return;
  const int key = static_cast<int>(idx / V);
  const int64_t sg0 = sgoff[n], nseg = sgoff[n + 1] - sg0;
  const int64_t o = (static_cast<int64_t>(n) * H + h) * KV + idx;
  float S = h0 ? h0[o] : 0.f;
  for (int64_t s = 0; s < nseg; ++s) {
    sin_[((sg0 + n + s) * H + h) * KV + idx] = S;
    S = cexp2(dtot[((sg0 + s) * H + h) * KD + key]) * S + eloc[((sg0 + s) * H + h) * KV + idx];
  }
  sin_[((sg0 + n + nseg) * H + h) * KV + idx] = S;
  float dS = dht ? dht[o] : 0.f;
  for (int64_t s = nseg - 1; s >= 0; --s) {
    dsend[((sg0 + s) * H + h) * KV + idx] = dS;
    const int64_t cf = coff[n] + s * kSegC;
    dS = cexp2(dtot[((sg0 + s) * H + h) * KD + key]) * dS + dloc[(cf * H + h) * KV + idx];
  }
  if (dh0) dh0[o] = dS;
}

// ------------------------------------------------------------ chunk pass --
// One workgroup (8 wavefronts) per (chunk, head).  Wavefronts w and w + 4
// own rows 16 I .. 16 I + 15 (I = w % 4) and split the output tiles between
// them (half P = w / 4): column blocks J of A and dA with J % 2 == P, key
// tiles 2 P and 2 P + 1 of dq and dk, value tiles N % 2 == P of dv; two
// wavefronts per SIMD hide each other's LDS latency.  dg is a reverse cumsum
// over the chunk.  q, k, v, do are staged as rows of 64 input-dtype values
// (value columns padded with zeros to VP = V rounded up to 32).
constexpr int kCW = 8;   // wavefronts per chunk workgroup
constexpr int kL16 = 64, kL32 = 64;   // LDS row lengths (16-bit and fp32 tiles)

struct __align__(16) SmemC {
  uint16_t q[BT][kL16], k[BT][kL16], v[BT][kL16], dout[BT][kL16];
  float h[KD][kL32];   // h[c] as [key][value]
  float dh[KD][kL32];  // dh[c] as [key][value]
  union {
    struct {
      float A[BT][kL32], dA[BT][kL32];
    } p;
    float r[BT][kL32];   // q dq - k dk (after the products)
  } u;
  float G[BT][kL32];   // log2 cumsum
  float M[4][KD];      // block reference points
  float glast[KD];
  float term[KD];      // sum_v dh[c] h[c+1]
  float bsum[kCW][KD];
};

template <int DT, bool GF32>
__global__ __launch_bounds__(64 * kCW) void bwd_chunk_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const void *__restrict__ g, const uint16_t *__restrict__ dout, const int64_t *__restrict__ cu,
    const int64_t *__restrict__ coff, const int64_t *__restrict__ sgoff, int n_seq, int64_t T, int H, int V,
    float scale, const float *__restrict__ hloc, const float *__restrict__ dfw, const float *__restrict__ dloc,
    const float *__restrict__ drv, const float *__restrict__ sin_, const float *__restrict__ dsend,
    uint16_t *__restrict__ dq, uint16_t *__restrict__ dk, uint16_t *__restrict__ dv, void *__restrict__ dg) {
  constexpr bool EX = DT == SSLA_BF16;   // input values are exact bf16 operands
  __shared__ SmemC sm;
  auto X = [](uint16_t b) { return Elt<DT>::f(b); };   // a staged input value
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int I = w & 3, P = w >> 2;
  const int h = static_cast<int>(blockIdx.x % H);
  const int64_t c = blockIdx.x / H;
  if (c >= coff[n_seq]) return;   // workgroup-uniform
  const int n = find_seq(coff, n_seq, c);
  int64_t bos, eos;
  seq_bounds(cu, n, T, bos, eos);
  const int64_t j = c - coff[n];
  const int64_t t0 = bos + j * BT;
  const int nrows = static_cast<int>(min(static_cast<int64_t>(BT), eos - t0));
  const int64_t KV = static_cast<int64_t>(KD) * V;
  const int VP = (V + 31) & ~31;
  // states of this chunk: local part + 2^decay * carried part (per key)
  const int64_t nc = (eos - bos + BT - 1) / BT;
  const int64_t sgi = sgoff[n] + j / kSegC;
  const bool last_in_seg = (j % kSegC) == kSegC - 1 || j == nc - 1;
  const float *sin_c = sin_ + ((sgi + n) * H + h) * KV;        // carried into this segment
  const float *sin_n = sin_ + ((sgi + n + 1) * H + h) * KV;    // carried into the next (or ht)
  const float *dsend_c = dsend + (sgi * H + h) * KV;           // gradient at this segment's end

  // ---- staging: q, k, v, do and the gates, 16-byte pieces from every thread
  {
    const uint4 z = {0, 0, 0, 0};
    auto put = [](void *dst, const uint4 &x) {   // 16 bytes into an 8-byte-aligned row
      uint2 *d = static_cast<uint2 *>(dst);
      d[0] = make_uint2(x.x, x.y);
      d[1] = make_uint2(x.z, x.w);
    };
    const int r = tid >> 3, pc = tid & 7;   // 64 rows x 8 pieces
    const int64_t oq = ((t0 + r) * H + h) * KD + pc * 8;
    put(&sm.q[r][pc * 8], r < nrows ? *reinterpret_cast<const uint4 *>(q + oq) : z);
    put(&sm.k[r][pc * 8], r < nrows ? *reinterpret_cast<const uint4 *>(k + oq) : z);
    const bool okv = r < nrows && pc * 8 < V;
    const int64_t ov = ((t0 + r) * H + h) * V + pc * 8;
    put(&sm.v[r][pc * 8], okv ? *reinterpret_cast<const uint4 *>(v + ov) : z);
    put(&sm.dout[r][pc * 8], okv ? *reinterpret_cast<const uint4 *>(dout + ov) : z);
    if constexpr (GF32) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid * 2 + i, rr = e >> 4, p4 = e & 15;
        put(&sm.G[rr][p4 * 4],
            rr < nrows
                ? *reinterpret_cast<const uint4 *>(static_cast<const float *>(g) + ((t0 + rr) * H + h) * KD + p4 * 4)
                : z);
      }
    } else {
      const uint4 u4 = r < nrows ? *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(g) + oq) : z;
      const uint16_t *u = reinterpret_cast<const uint16_t *>(&u4);
#pragma unroll
      for (int qq = 0; qq < 8; ++qq) sm.G[r][pc * 8 + qq] = Elt<DT>::f(u[qq]);
    }
  }
  {   // h[c], dh[c] (leaving-state gradient) and sum_v dh[c] h[c+1]; row = key,
      // 8 threads per key, 8 value columns each (float4 pieces)
    const int key = tid >> 3, c0 = (tid & 7) * 8;
    const float fe = cexp2(dfw[(c * H + h) * KD + key]);
    const float fn = last_in_seg ? 0.f : cexp2(dfw[((c + 1) * H + h) * KD + key]);
    const float fr = last_in_seg ? 0.f : cexp2(drv[((c + 1) * H + h) * KD + key]);
    float part = 0.f;
#pragma unroll
    for (int e4 = 0; e4 < 8; e4 += 4) {
      const int vc = c0 + e4;
      float4 hv = {0.f, 0.f, 0.f, 0.f}, dv4 = {0.f, 0.f, 0.f, 0.f};
      if (vc < V) {
        const int64_t o = static_cast<int64_t>(key) * V + vc;
        const float4 sc = *reinterpret_cast<const float4 *>(sin_c + o);
        const float4 hl = *reinterpret_cast<const float4 *>(hloc + (c * H + h) * KV + o);
        hv = make_float4(hl.x + fe * sc.x, hl.y + fe * sc.y, hl.z + fe * sc.z, hl.w + fe * sc.w);
        float4 hn, ds = *reinterpret_cast<const float4 *>(dsend_c + o);
        if (last_in_seg) {
          hn = *reinterpret_cast<const float4 *>(sin_n + o);
          dv4 = ds;
        } else {
          const float4 hl1 = *reinterpret_cast<const float4 *>(hloc + ((c + 1) * H + h) * KV + o);
          const float4 dl1 = *reinterpret_cast<const float4 *>(dloc + ((c + 1) * H + h) * KV + o);
          hn = make_float4(hl1.x + fn * sc.x, hl1.y + fn * sc.y, hl1.z + fn * sc.z, hl1.w + fn * sc.w);
          dv4 = make_float4(dl1.x + fr * ds.x, dl1.y + fr * ds.y, dl1.z + fr * ds.z, dl1.w + fr * ds.w);
        }
        part += dv4.x * hn.x + dv4.y * hn.y + dv4.z * hn.z + dv4.w * hn.w;
      }
      *reinterpret_cast<float2 *>(&sm.h[key][vc]) = make_float2(hv.x, hv.y);
      *reinterpret_cast<float2 *>(&sm.h[key][vc + 2]) = make_float2(hv.z, hv.w);
      *reinterpret_cast<float2 *>(&sm.dh[key][vc]) = make_float2(dv4.x, dv4.y);
      *reinterpret_cast<float2 *>(&sm.dh[key][vc + 2]) = make_float2(dv4.z, dv4.w);
    }
    part += __shfl_xor(part, 1);
    part += __shfl_xor(part, 2);
    part += __shfl_xor(part, 4);
    if ((tid & 7) == 0) sm.term[key] = part;
  }
  __syncthreads();
  gate_cumsum<64 * kCW>(sm.G, sm.bsum, sm.glast);   // (bsum doubles as its scratch)
  if (w == 0) {   // block reference points
    float ep = 0.f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float eb = sm.G[b * 16 + 15][lane];
      sm.M[b][lane] = 0.5f * (ep + eb);
      ep = eb;
    }
  }
  __syncthreads();

  // ---- A and dA, rows of block I, column blocks J of this half (zero above
  // the diagonal); the q side (q e^(G - M_I)) is the same for every J
  {
    float qa[2][8];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kk = ks * 32 + grp * 8 + e, t = 16 * I + col;
        qa[ks][e] = X(sm.q[t][kk]) * cexp2(sm.G[t][kk] - sm.M[I][kk]);
      }
    for (int J = P; J < 4; J += 2) {
      f32x4 a4 = {0.f, 0.f, 0.f, 0.f}, d4 = {0.f, 0.f, 0.f, 0.f};
      if (J <= I) {
        const int t = 16 * I + col, s = 16 * J + col;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          float b[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int kk = ks * 32 + grp * 8 + e;
            b[e] = X(sm.k[s][kk]) * cexp2(sm.M[I][kk] - sm.G[s][kk]);
          }
          a4 = mmax<false, false>(qa[ks], b, a4);
        }
        for (int vs = 0; vs < VP; vs += 32) {
          float a[8], b[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int vc = vs + grp * 8 + e;
            a[e] = X(sm.dout[t][vc]);
            b[e] = X(sm.v[s][vc]);
          }
          d4 = mmax<EX, EX>(a, b, d4);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * I + grp * 4 + i, s = 16 * J + col;
        const bool keep = J <= I && s <= t;
        sm.u.p.A[t][s] = keep ? scale * a4[i] : 0.f;
        sm.u.p.dA[t][s] = keep ? scale * d4[i] : 0.f;
      }
    }
  }
  __syncthreads();

  // ---- dq (rows t of block I), key tiles 2P, 2P + 1
  float dqv[2][4], dkv[2][4];
  {
    f32x4 ai[2], ae[2];
#pragma unroll
    for (int nn = 0; nn < 2; ++nn) {
      ai[nn] = f32x4{0.f, 0.f, 0.f, 0.f};
      ae[nn] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int t = 16 * I + col;
    const int s_end = 16 * (I + 1);
    for (int ss = 0; ss < s_end; ss += 32) {   // intra: dA[t, s] (k e^(M_I - G))[s, key]
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = sm.u.p.dA[t][ss + grp * 8 + e];
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        const int key = (2 * P + nn) * 16 + col;
        const float m = sm.M[I][key];
        float b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int s = ss + grp * 8 + e;
          b[e] = s < s_end ? X(sm.k[s][key]) * cexp2(m - sm.G[s][key]) : 0.f;
        }
        ai[nn] = mmax<false, false>(a, b, ai[nn]);
      }
    }
    for (int vs = 0; vs < VP; vs += 32) {   // inter: do[t, v] h[c][key, v]
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = X(sm.dout[t][vs + grp * 8 + e]);
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        const int key = (2 * P + nn) * 16 + col;
        float b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) b[e] = sm.h[key][vs + grp * 8 + e];
        ae[nn] = mmax<EX, false>(a, b, ae[nn]);
      }
    }
#pragma unroll
    for (int nn = 0; nn < 2; ++nn)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tt = 16 * I + grp * 4 + i, key = (2 * P + nn) * 16 + col;
        const float gt = sm.G[tt][key];
        dqv[nn][i] = ai[nn][i] * cexp2(gt - sm.M[I][key]) + scale * ae[nn][i] * cexp2(gt);
      }
  }
  // ---- dk (rows s of block I), key tiles 2P, 2P + 1
  {
    f32x4 ai[2], ae[2];
#pragma unroll
    for (int nn = 0; nn < 2; ++nn) {
      ai[nn] = f32x4{0.f, 0.f, 0.f, 0.f};
      ae[nn] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int s = 16 * I + col;
    const int t_beg = 16 * I;
    for (int ts = t_beg & ~31; ts < BT; ts += 32) {   // intra: dA[t, s] (q e^(G - M_I))[t, key]
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = sm.u.p.dA[ts + grp * 8 + e][s];
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        const int key = (2 * P + nn) * 16 + col;
        const float m = sm.M[I][key];
        float b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int t = ts + grp * 8 + e;
          b[e] = t >= t_beg ? X(sm.q[t][key]) * cexp2(sm.G[t][key] - m) : 0.f;
        }
        ai[nn] = mmax<false, false>(a, b, ai[nn]);
      }
    }
    for (int vs = 0; vs < VP; vs += 32) {   // inter: v[s, v] dh[c][key, v]
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = X(sm.v[s][vs + grp * 8 + e]);
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        const int key = (2 * P + nn) * 16 + col;
        float b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) b[e] = sm.dh[key][vs + grp * 8 + e];
        ae[nn] = mmax<EX, false>(a, b, ae[nn]);
      }
    }
#pragma unroll
    for (int nn = 0; nn < 2; ++nn)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ss = 16 * I + grp * 4 + i, key = (2 * P + nn) * 16 + col;
        const float gs = sm.G[ss][key];
        dkv[nn][i] = ai[nn][i] * cexp2(sm.M[I][key] - gs) + ae[nn][i] * cexp2(sm.glast[key] - gs);
      }
  }
  // ---- dv (rows s of block I), value tiles N with N % 2 == P
  for (int N = P; N < VP / 16; N += 2) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int s = 16 * I + col;
    const int vc = N * 16 + col;
    const int t_beg = 16 * I;
    for (int ts = t_beg & ~31; ts < BT; ts += 32) {   // intra: A[t, s] do[t, v]
      float a[8], b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = ts + grp * 8 + e;
        a[e] = sm.u.p.A[t][s];
        b[e] = X(sm.dout[t][vc]);
      }
      acc = mmax<false, EX>(a, b, acc);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {   // inter: (k e^(G_last - G))[s, key] dh[c][key, v]
      float a[8], b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kk = ks * 32 + grp * 8 + e;
        a[e] = X(sm.k[s][kk]) * cexp2(sm.glast[kk] - sm.G[s][kk]);
        b[e] = sm.dh[kk][vc];
      }
      acc = mmax<false, false>(a, b, acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ss = 16 * I + grp * 4 + i, vcc = N * 16 + col;
      if (ss < nrows && vcc < V) dv[((t0 + ss) * H + h) * V + vcc] = Elt<DT>::b(acc[i]);
    }
  }
  // ---- dq, dk out; r = q dq - k dk for dg
  __syncthreads();   // every wavefront is done with A and dA (r reuses them)
#pragma unroll
  for (int nn = 0; nn < 2; ++nn)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tt = 16 * I + grp * 4 + i, key = (2 * P + nn) * 16 + col;
      sm.u.r[tt][key] = X(sm.q[tt][key]) * dqv[nn][i] - X(sm.k[tt][key]) * dkv[nn][i];
      if (tt < nrows) {
        const int64_t o = ((t0 + tt) * H + h) * KD + key;
        dq[o] = Elt<DT>::b(dqv[nn][i]);
        dk[o] = Elt<DT>::b(dkv[nn][i]);
      }
    }
  __syncthreads();
  // ---- dg: reverse cumsum over the chunk + the leaving-state term;
  // thread (w, lane): key = lane, rows 8 w .. 8 w + 7
  {
    const int key = lane;
    float sacc = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) sacc += sm.u.r[8 * w + r][key];
    sm.bsum[w][key] = sacc;
    __syncthreads();
    float run = sm.term[key];
    for (int b = kCW - 1; b > w; --b) run += sm.bsum[b][key];
#pragma unroll
    for (int r = 7; r >= 0; --r) {
      const int tt = 8 * w + r;
      run += sm.u.r[tt][key];
      if (tt < nrows) {
        const int64_t o = ((t0 + tt) * H + h) * KD + key;
        if constexpr (GF32) static_cast<float *>(dg)[o] = run;
        else static_cast<uint16_t *>(dg)[o] = Elt<DT>::b(run);
      }
    }
  }
}

// Workspace: offsets, per-chunk local states / decays of both passes, and
// per-segment end states, decays, carried states and gradients.
struct BwdWs {
  int64_t *coff, *sgoff;
  float *hloc, *dloc, *dfw, *drv, *eloc, *dtot, *sin_, *dsend;
  size_t total;
};
inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
inline BwdWs bwd_ws(char *base, int n_seq, int64_t T, int H, int V) {
  const int64_t cmax = (T + BT - 1) / BT + n_seq;                  // chunks
  const int64_t smax = (cmax + kSegC - 1) / kSegC + n_seq;         // segments
  const size_t kv = static_cast<size_t>(H) * KD * V * sizeof(float), kk = static_cast<size_t>(H) * KD * sizeof(float);
  BwdWs w;
  size_t p = 0;
  auto take = [&](size_t bytes) {
    char *q = base ? base + p : nullptr;
    p = align256(p + bytes);
    return q;
  };
  w.coff = reinterpret_cast<int64_t *>(take(sizeof(int64_t) * (n_seq + 1)));
  w.sgoff = reinterpret_cast<int64_t *>(take(sizeof(int64_t) * (n_seq + 1)));
  w.hloc = reinterpret_cast<float *>(take(kv * cmax));
  w.dloc = reinterpret_cast<float *>(take(kv * cmax));
  w.dfw = reinterpret_cast<float *>(take(kk * cmax));
  w.drv = reinterpret_cast<float *>(take(kk * cmax));
  w.eloc = reinterpret_cast<float *>(take(kv * smax));
  w.dtot = reinterpret_cast<float *>(take(kk * smax));
  w.sin_ = reinterpret_cast<float *>(take(kv * (smax + n_seq)));
  w.dsend = reinterpret_cast<float *>(take(kv * smax));
  w.total = p;
  return w;
}

template <int DT, bool GF32>
int launch_bwd(const void *q, const void *k, const void *v, const void *g, const int64_t *cu, int n_seq, int64_t T,
               int H, int V, float scale, const float *h0, const void *dout, const float *dht, void *dq, void *dk,
               void *dv, void *dg, float *dh0, const BwdWs &w, hipStream_t st) {
  const auto *Q = static_cast<const uint16_t *>(q);
  const auto *Kp = static_cast<const uint16_t *>(k);
  const auto *Vp = static_cast<const uint16_t *>(v);
  const auto *DO = static_cast<const uint16_t *>(dout);
  hipLaunchKernelGGL(bwd_offsets_kernel, dim3(1), dim3(256), 0, st, cu, n_seq, T, w.coff, w.sgoff);
  const int64_t cmax = (T + BT - 1) / BT + n_seq;
  const int64_t smax = (cmax + kSegC - 1) / kSegC + n_seq;
  const int64_t nb = smax * H;
  hipLaunchKernelGGL((bwd_seg_passes<DT, GF32>), dim3(static_cast<unsigned>(2 * nb)), dim3(256), 0, st, Kp, Vp, Q, DO,
                     g, cu, w.coff, w.sgoff, n_seq, T, H, V, scale, nb, w.hloc, w.dfw, w.eloc, w.dtot, w.dloc, w.drv);
  const int64_t fold_threads = static_cast<int64_t>(n_seq) * H * KD * V;
  hipLaunchKernelGGL(bwd_fold_kernel, dim3(static_cast<unsigned>((fold_threads + 255) / 256)), dim3(256), 0, st,
                     w.coff, w.sgoff, n_seq, H, V, h0, dht, w.eloc, w.dtot, w.dloc, w.sin_, w.dsend, dh0);
  hipLaunchKernelGGL((bwd_chunk_kernel<DT, GF32>), dim3(static_cast<unsigned>(cmax * H)), dim3(64 * kCW), 0, st, Q, Kp, Vp,
                     g, DO, cu, w.coff, w.sgoff, n_seq, T, H, V, scale, w.hloc, w.dfw, w.dloc, w.drv, w.sin_,
                     w.dsend, static_cast<uint16_t *>(dq), static_cast<uint16_t *>(dk), static_cast<uint16_t *>(dv),
                     dg);
  return launch_status("gla_chunk_bwd");
}

// With no rows at all (T == 0) every sequence is empty: its initial-state
// gradient is the final-state gradient (ht == h0), or zero without one.
__global__ __launch_bounds__(256) void bwd_empty_dh0_kernel(const float *__restrict__ dht, float *__restrict__ dh0,
                                                            int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dh0[i] = dht ? dht[i] : 0.f;
}

}  // namespace
}  // namespace ssla

extern "C" size_t ssla_gla_chunk_bwd_workspace_size(int n_seq, int64_t T, int H, int K, int V) {
  if (n_seq < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0) return 0;
  return ssla::bwd_ws(nullptr, n_seq, T, H, V).total;
}

extern "C" int ssla_gla_chunk_bwd(const void *q, const void *k, const void *v, const void *g, int g_dtype,
                                  const int64_t *cu_seqlens, int n_seq, int64_t T, int H, int K, int V,
                                  float scale, const float *h0, const void *dout, const float *dht, void *dq,
                                  void *dk, void *dv, void *dg, float *dh0, int dtype, void *workspace,
                                  size_t workspace_bytes, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && T >= 0 && H > 0, "gla_chunk_bwd: bad sizes n_seq=%d T=%lld H=%d", n_seq,
                 (long long)T, H);
  if (dtype != SSLA_BF16 && dtype != SSLA_F16) {
    set_error("gla_chunk_bwd: dtype must be BF16 or F16");
    return SSLA_ERR_DTYPE;
  }
  if (g_dtype != SSLA_F32 && g_dtype != dtype) {
    set_error("gla_chunk_bwd: g must be F32 or the input dtype");
    return SSLA_ERR_DTYPE;
  }
  if (K != KD || V % 16 != 0 || V <= 0 || V > 64) {
    set_error("gla_chunk_bwd: needs K == 64 and V a multiple of 16 up to 64 (K=%d V=%d)", K, V);
    return SSLA_ERR_UNSUPPORTED;
  }
  if (n_seq == 0) return SSLA_OK;
  if (T == 0) {
    if (!dh0) return SSLA_OK;
    const int64_t n = static_cast<int64_t>(n_seq) * H * K * V;
    hipLaunchKernelGGL(bwd_empty_dh0_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), dht, dh0, n);
    return launch_status("gla_chunk_bwd");
  }
  SSLA_CHECK_ARG(q && k && v && g && cu_seqlens && dout && dq && dk && dv && dg, "gla_chunk_bwd: null pointer");
  const size_t need = ssla_gla_chunk_bwd_workspace_size(n_seq, T, H, K, V);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("gla_chunk_bwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(aligned(workspace, 16), "gla_chunk_bwd: workspace must be 16-byte aligned");
  const int64_t chunks = (T + BT - 1) / BT + n_seq;
  if (chunks * H > 0x7fffffff) {
    set_error("gla_chunk_bwd: too many chunks");
    return SSLA_ERR_UNSUPPORTED;
  }
  const BwdWs w = bwd_ws(static_cast<char *>(workspace), n_seq, T, H, V);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool gf32 = g_dtype == SSLA_F32;
  if (dtype == SSLA_BF16)
    return gf32 ? launch_bwd<SSLA_BF16, true>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, dout, dht, dq, dk,
                                              dv, dg, dh0, w, st)
                : launch_bwd<SSLA_BF16, false>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, dout, dht, dq,
                                               dk, dv, dg, dh0, w, st);
  return gf32 ? launch_bwd<SSLA_F16, true>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, dout, dht, dq, dk, dv,
                                           dg, dh0, w, st)
              : launch_bwd<SSLA_F16, false>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, dout, dht, dq, dk,
                                            dv, dg, dh0, w, st);
}
