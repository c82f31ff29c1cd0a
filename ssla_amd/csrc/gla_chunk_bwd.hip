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
#include "lds_tile.h"

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
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wavefront-uniform
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
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wavefront-uniform
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

// ------------------------------------------------------ walking chunk pass --
// bf16 inputs: one workgroup (8 wavefronts) per (segment, head) walks the
// segment's chunks in order and carries the state h (fp32, in registers)
// from the segment's carried entering state, so the forward local pass
// stores no per-chunk states; dh of each chunk is the reverse pass's local
// gradient plus the decayed end gradient of the segment.  Per chunk the
// operands are staged once in LDS as swizzled bf16 tiles (the decay-scaled
// ones, h and dh as hi / lo pairs) and every product reads them there;
// the next chunk's inputs load into registers meanwhile.
//
// Wavefront w: I = w % 4, P = w / 4; lane = 16 gq + r.  It owns rows
// 16 I + r (as t of dq and s of dk, dv, dg), key tiles / value tiles 2P and
// 2P + 1 of its outputs, and state keys 16 I .. 16 I + 15 (value tiles 2P,
// 2P + 1).  A 16 x 16 MFMA result C[m][n] sits in the lanes as (m = 4 gq + i,
// n = r): the operand layout of a 16x16x16 MFMA with n = r and k = m, so the
// dA^T (for dq), dA (for dk) and A (for dv) blocks this wavefront computes
// feed the next products from registers.
//
// Decay references as in the other passes (log2 units, E_I = G at the last
// row of block I, M_I its midpoint with E_-1 = 0): diagonal blocks use
// q 2^(G - M_I) and k 2^(M_I - G); blocks t in I' > s in I use q 2^(G - M_I'),
// k 2^(E_I - G) and the per-key factor 2^(M_I' - E_I) <= 1.
constexpr int kWW = 8;           // wavefronts of the walking kernel
constexpr int kGP = 68;          // fp32 G row pitch (floats)

struct __align__(16) SmemW {
  uint16_t q[64 * 64], k[64 * 64], v[64 * 64], dout[64 * 64];   // raw bf16 rows
  uint16_t qm[2][64 * 64];   // q 2^(G - M_I)          hi, lo
  uint16_t km[2][64 * 64];   // k 2^(M_I - G)
  uint16_t ke[2][64 * 64];   // k 2^(E_I - G)
  uint16_t kb[2][64 * 64];   // k 2^(gamma - G)
  uint16_t h[2][64 * 64];    // h[c], [key][value]
  uint16_t dh[2][64 * 64];   // dh[c], [key][value]
  float G[BT][kGP];          // log2 cumsum, [row][key]
  float M[4][KD], E[4][KD];
  float Fe[4][4][KD];        // 2^(M_I' - E_I), I' > I
  float gam[KD], dgam[KD], hdh[KD];
  float psum[kWW][KD];
  float btot[2][4][KD];      // per-block totals: sum of dG, sum of tdk
};

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ float row_shl(float x) {   // lane i <- lane i + N of its 16-lane row (0 past the row)
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x100 + N, 0xf, 0xf, true));
}

__device__ __forceinline__ f32x4 mma16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// x = hi + lo to about 2^-16 relative, in packed pairs: one conversion per
// two values and one shift or mask per value to widen the head back
__device__ __forceinline__ uint32_t cvt2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}
__device__ __forceinline__ float lo_half(uint32_t p) { return __builtin_bit_cast(float, p << 16); }
__device__ __forceinline__ float hi_half(uint32_t p) { return __builtin_bit_cast(float, p & 0xffff0000u); }
template <int N>
__device__ __forceinline__ void split_pairs(const float *x, uint32_t *hi, uint32_t *lo) {
#pragma unroll
  for (int j = 0; j < N / 2; ++j) {
    hi[j] = cvt2(x[2 * j], x[2 * j + 1]);
    lo[j] = cvt2(x[2 * j] - lo_half(hi[j]), x[2 * j + 1] - hi_half(hi[j]));
  }
}
__device__ __forceinline__ void split4(f32x4 x, s16x4 &hi, s16x4 &lo) {
  const float v[4] = {x[0], x[1], x[2], x[3]};
  uint32_t h[2], l[2];
  split_pairs<4>(v, h, l);
  hi = __builtin_bit_cast(s16x4, make_uint2(h[0], h[1]));
  lo = __builtin_bit_cast(s16x4, make_uint2(l[0], l[1]));
}
__device__ __forceinline__ void split8(f32x8 x, bf16x8 &hi, bf16x8 &lo) {
  const float v[8] = {x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
  uint32_t h[4], l[4];
  split_pairs<8>(v, h, l);
  hi = __builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3]));
  lo = __builtin_bit_cast(bf16x8, make_uint4(l[0], l[1], l[2], l[3]));
}
__device__ __forceinline__ f32x8 widen8(const uint4 &b) {
  return f32x8{lo_half(b.x), hi_half(b.x), lo_half(b.y), hi_half(b.y),
               lo_half(b.z), hi_half(b.z), lo_half(b.w), hi_half(b.w)};
}
__device__ __forceinline__ f32x4 widen4(const uint2 &b) {
  return f32x4{lo_half(b.x), hi_half(b.x), lo_half(b.y), hi_half(b.y)};
}
__device__ __forceinline__ uint2 pack4(f32x4 x) { return make_uint2(cvt2(x[0], x[1]), cvt2(x[2], x[3])); }
__device__ __forceinline__ f32x4 ld4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }
// x, or zeros when !ok, component-wise (a select of whole uint4 / f32x4
// values can turn the registers holding them into scratch memory)
__device__ __forceinline__ uint4 keep4(const uint4 &x, bool ok) {
  const uint32_t mk = ok ? 0xffffffffu : 0u;
  return make_uint4(x.x & mk, x.y & mk, x.z & mk, x.w & mk);
}
__device__ __forceinline__ float keep1(float v, uint32_t mk) {
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) & mk);
}
// (the elements go through scalars: a bit cast of a vector element itself
// reads the vector's first element)
__device__ __forceinline__ f32x4 keepf4(const f32x4 &x, bool ok) {
  const uint32_t mk = ok ? 0xffffffffu : 0u;
  return f32x4{keep1(x[0], mk), keep1(x[1], mk), keep1(x[2], mk), keep1(x[3], mk)};
}

// ------------------------------------------- state passes on staged tiles --
// bf16 inputs: the local passes of the walking path.  One workgroup (4
// wavefronts) per (segment, head) runs a segment from a zero state; per
// chunk the decay-scaled X tile (hi / lo) and the raw Y tile are staged once
// and wavefront w accumulates value columns 16 w .. 16 w + 15 of all 64 keys
// (lane: keys 16 kb + 4 gq + i, column 16 w + r):
// * forward: X = k, Y = v, X~ = k 2^(gamma - G); keeps only the segment's
//   end state and total decay (the walking chunk pass carries the state);
// * reverse: X = scale q, Y = do, X~ = scale q 2^G, chunks in reverse;
//   stores the local gradient of the state entering each chunk and the log2
//   decay from there to the segment end.
struct __align__(16) SmemT {
  uint16_t xt[2][64 * 64];   // X~ hi, lo
  uint16_t x[64 * 64], y[64 * 64];
  float G[BT][kGP];
  float gam[KD], dgam[KD];
  float psum[4][KD];
};

template <bool REV, bool GF32>
__device__ __forceinline__ void seg_pass_tiles(SmemT &sm, const int64_t bid, const uint16_t *__restrict__ X,
                                               const uint16_t *__restrict__ Y, const void *__restrict__ g,
                                               const int64_t *__restrict__ cu, const int64_t *__restrict__ coff,
                                               const int64_t *__restrict__ sgoff, int n_seq, int64_t T, int H, int V,
                                               float xscale, float *__restrict__ loc, float *__restrict__ dec,
                                               float *__restrict__ eloc, float *__restrict__ dtot) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wavefront-uniform
  const int h = static_cast<int>(bid % H);
  const int64_t sg = bid / H;
  if (sg >= sgoff[n_seq]) return;   // workgroup-uniform
  const int n = find_seq(sgoff, n_seq, sg);
  int64_t bos, eos;
  seq_bounds(cu, n, T, bos, eos);
  const int64_t nc = (eos - bos + BT - 1) / BT;
  const int64_t j0 = (sg - sgoff[n]) * kSegC;
  const int m = static_cast<int>(min(static_cast<int64_t>(kSegC), nc - j0));
  const int64_t c0 = coff[n] + j0;
  const int v0 = 16 * w;
  const bool active = v0 < V;
  const int64_t KV = static_cast<int64_t>(KD) * V;

  // pieces: 16-bit rows pr and pr + 32 (columns pc .. pc + 7); fp32 g rows
  // fr + 16 u (columns fc .. fc + 3)
  const int pr = tid >> 3, pc = 8 * (tid & 7);
  const int fr = tid >> 4, fc = 4 * (tid & 15);
  uint4 px[2], py[2], pg16[2];
  f32x4 pg[4];
  // Loads go to clamped (always valid) addresses and rows past the chunk /
  // columns past V are zeroed when staged: a select right after a load
  // would make the compiler wait for it at once.
  auto fetch = [&](int64_t j) {
    const int64_t t0 = bos + j * BT;
    const int last = static_cast<int>(min(static_cast<int64_t>(BT), eos - t0)) - 1;
    const int pcv = pc < V ? pc : 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t o = (t0 + min(pr + 32 * u, last)) * H + h;
      px[u] = *reinterpret_cast<const uint4 *>(X + o * KD + pc);
      py[u] = *reinterpret_cast<const uint4 *>(Y + o * V + pcv);
      if constexpr (!GF32) pg16[u] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(g) + o * KD + pc);
    }
    if constexpr (GF32) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        pg[u] = ld4(static_cast<const float *>(g) + ((t0 + min(fr + 16 * u, last)) * H + h) * KD + fc);
    }
  };

  f32x4 acc[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) acc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float D = 0.f;   // wavefront 0, lane = key: log2 decay so far
  const int r = lane & 15, gq = lane >> 4;
  auto store_loc = [&](int64_t c) {
    if (!loc) return;
    if (active) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          loc[(c * H + h) * KV + static_cast<int64_t>(kb * 16 + gq * 4 + i) * V + v0 + r] = acc[kb][i];
    }
    if (w == 0) dec[(c * H + h) * KD + lane] = D;
  };

  fetch(REV ? j0 + m - 1 : j0);
  for (int it = 0; it < m; ++it) {
    const int64_t j = REV ? j0 + m - 1 - it : j0 + it;
    const int nrows = static_cast<int>(min(static_cast<int64_t>(BT), eos - (bos + j * BT)));
    // ---- raw X, Y and g into LDS; then the next chunk's loads
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bool ok = pr + 32 * u < nrows;
      tile_store8(sm.x, pr + 32 * u, pc, keep4(px[u], ok));
      tile_store8(sm.y, pr + 32 * u, pc, keep4(py[u], ok && pc < V));
    }
    if constexpr (GF32) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        *reinterpret_cast<f32x4 *>(&sm.G[fr + 16 * u][fc]) = keepf4(pg[u], fr + 16 * u < nrows);
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f32x8 gv = widen8(keep4(pg16[u], pr + 32 * u < nrows));
        *reinterpret_cast<f32x4 *>(&sm.G[pr + 32 * u][pc]) = f32x4{gv[0], gv[1], gv[2], gv[3]};
        *reinterpret_cast<f32x4 *>(&sm.G[pr + 32 * u][pc + 4]) = f32x4{gv[4], gv[5], gv[6], gv[7]};
      }
    }
    if (it + 1 < m) fetch(REV ? j - 1 : j + 1);
    lds_barrier();
    // ---- log2 cumsum per key: thread (key, 16-row quarter)
    {
      const int key = tid & 63, rq = tid >> 6;
      float run[16], s = 0.f;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        s += sm.G[16 * rq + rr][key];
        run[rr] = s;
      }
      sm.psum[rq][key] = s;
      lds_barrier();
      float off = 0.f;
      for (int b = 0; b < rq; ++b) off += sm.psum[b][key];
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) sm.G[16 * rq + rr][key] = (run[rr] + off) * kLog2e;
      if (rq == 3) {
        const float gm = (s + off) * kLog2e;
        sm.gam[key] = gm;
        sm.dgam[key] = cexp2(gm);
      }
    }
    lds_barrier();
    // ---- X~ (hi / lo)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int rr = pr + 32 * u;
      const f32x8 xf = widen8(tile_row8(sm.x, rr, pc));
      f32x8 xs;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float G = sm.G[rr][pc + e];
        xs[e] = xf[e] * xscale * cexp2(REV ? G : sm.gam[pc + e] - G);
      }
      bf16x8 hi, lo;
      split8(xs, hi, lo);
      tile_store8(sm.xt[0], rr, pc, to_bits(hi));
      tile_store8(sm.xt[1], rr, pc, to_bits(lo));
    }
    lds_barrier();
    // ---- acc <- 2^gamma acc + X~^T Y
    if (active) {
      bf16x8 yb[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) yb[ks] = tr_operand<bf16x8>(sm.y, 32 * ks + 8 * gq, 32 * ks + 8 * gq + 4, v0, lane);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        acc[kb] *= ld4(&sm.dgam[16 * kb + 4 * gq]);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int ra = 32 * ks + 8 * gq;
          acc[kb] = mma32(tr_operand<bf16x8>(sm.xt[0], ra, ra + 4, 16 * kb, lane), yb[ks], acc[kb]);
          acc[kb] = mma32(tr_operand<bf16x8>(sm.xt[1], ra, ra + 4, 16 * kb, lane), yb[ks], acc[kb]);
        }
      }
    }
    D += sm.gam[lane];
    if (REV) store_loc(c0 + (j - j0));
    lds_barrier();   // the tiles are rewritten by the next chunk
  }
  if (!REV) {
    if (active) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          eloc[(sg * H + h) * KV + static_cast<int64_t>(kb * 16 + gq * 4 + i) * V + v0 + r] = acc[kb][i];
    }
    if (w == 0) dtot[(sg * H + h) * KD + lane] = D;
  }
}

// Both local passes in one launch (blocks [0, nb) forward, [nb, 2 nb) reverse).
template <bool GF32>
__global__ __launch_bounds__(256) void bwd_seg_passes_tiles(const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
                                                            const uint16_t *__restrict__ q,
                                                            const uint16_t *__restrict__ dout, const void *__restrict__ g,
                                                            const int64_t *__restrict__ cu,
                                                            const int64_t *__restrict__ coff,
                                                            const int64_t *__restrict__ sgoff, int n_seq, int64_t T,
                                                            int H, int V, float scale, int64_t nb,
                                                            float *__restrict__ eloc, float *__restrict__ dtot,
                                                            float *__restrict__ dloc, float *__restrict__ drv) {
  __shared__ SmemT sm;
  const int64_t b = blockIdx.x;
  if (b < nb)
    seg_pass_tiles<false, GF32>(sm, b, k, v, g, cu, coff, sgoff, n_seq, T, H, V, 1.f, nullptr, nullptr, eloc, dtot);
  else
    seg_pass_tiles<true, GF32>(sm, b - nb, q, dout, g, cu, coff, sgoff, n_seq, T, H, V, scale, dloc, drv, nullptr,
                               nullptr);
}

// Products and outputs of one chunk for wavefront (I, P) (phases 5-9 of
// bwd_walk_kernel); P is a template parameter so that the LDS addresses of
// its key and value tiles fold into immediate offsets.
template <bool GF32, int P>
__device__ __forceinline__ void walk_chunk(SmemW &sm, const int I, const int lane, const int nrows, const int64_t t0,
                                           const int H, const int h, const int V, const float scale, f32x4 (&hs)[2],
                                           uint16_t *__restrict__ dq, uint16_t *__restrict__ dk,
                                           uint16_t *__restrict__ dv, void *__restrict__ dg) {
  // lane indices through an opaque zero: otherwise the compiler hoists the
  // LDS addresses of every product out of the chunk loop and spills them
  int zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
  const int r = (lane & 15) + zero, gq = (lane >> 4) + zero;
  const int row = 16 * I + r;          // this lane's row (t or s)
  const bool row_ok = row < nrows;
  const int64_t orow = (t0 + row) * H + h;
  f32x4 dGv[2], tdk[2];

  // ---- (5) dq: dA^T blocks (s in J <= I, t in I), then per key tile
  {
    s16x4 dath[4], datl[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      if (J <= I) {
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          c = mma32(from_bits<bf16x8>(tile_row8(sm.v, 16 * J + r, 32 * ks + 8 * gq)),
                    from_bits<bf16x8>(tile_row8(sm.dout, row, 32 * ks + 8 * gq)), c);
        if (J == I) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (4 * gq + i > r) c[i] = 0.f;   // s > t
        }
        split4(c, dath[J], datl[J]);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int kt = 2 * P + u, kc = 16 * kt + 4 * gq;   // output keys kc .. kc + 3
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        if (J <= I) {
          const uint16_t *th = J == I ? sm.km[0] : sm.ke[0];
          const uint16_t *tl = J == I ? sm.km[1] : sm.ke[1];
          const s16x4 ah = tr_read4(th, 16 * J + 4 * gq, 16 * kt, lane);
          const s16x4 al = tr_read4(tl, 16 * J + 4 * gq, 16 * kt, lane);
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
          c = mma16(ah, dath[J], c);
          c = mma16(al, dath[J], c);
          c = mma16(ah, datl[J], c);
          if (J == I) acc += c;
          else acc += ld4(&sm.Fe[I][J][kc]) * c;
        }
      }
      f32x4 ci = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 d = from_bits<bf16x8>(tile_row8(sm.dout, row, 32 * ks + 8 * gq));
        ci = mma32(from_bits<bf16x8>(tile_row8(sm.h[0], 16 * kt + r, 32 * ks + 8 * gq)), d, ci);
        ci = mma32(from_bits<bf16x8>(tile_row8(sm.h[1], 16 * kt + r, 32 * ks + 8 * gq)), d, ci);
      }
      const f32x4 G4 = ld4(&sm.G[row][kc]), M4 = ld4(&sm.M[I][kc]);
      f32x4 dqv;
#pragma unroll
      for (int i = 0; i < 4; ++i) dqv[i] = scale * fmaf(cexp2(G4[i] - M4[i]), acc[i], cexp2(G4[i]) * ci[i]);
      dGv[u] = widen4(tile_row4(sm.q, row, kc)) * dqv;
      if (row_ok) *reinterpret_cast<uint2 *>(dq + orow * KD + kc) = pack4(dqv);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // ---- (6) dk: dA blocks (t in I' >= I, s in I), then per key tile
  {
    s16x4 dah[4], dal[4];
#pragma unroll
    for (int Ip = 0; Ip < 4; ++Ip) {
      if (Ip >= I) {
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          c = mma32(from_bits<bf16x8>(tile_row8(sm.dout, 16 * Ip + r, 32 * ks + 8 * gq)),
                    from_bits<bf16x8>(tile_row8(sm.v, row, 32 * ks + 8 * gq)), c);
        if (Ip == I) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (r > 4 * gq + i) c[i] = 0.f;   // s > t
        }
        split4(c, dah[Ip], dal[Ip]);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int kt = 2 * P + u, kc = 16 * kt + 4 * gq;
      f32x4 ad = {0.f, 0.f, 0.f, 0.f}, ao = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int Ip = 0; Ip < 4; ++Ip) {
        if (Ip >= I) {
          const s16x4 ah = tr_read4(sm.qm[0], 16 * Ip + 4 * gq, 16 * kt, lane);
          const s16x4 al = tr_read4(sm.qm[1], 16 * Ip + 4 * gq, 16 * kt, lane);
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
          c = mma16(ah, dah[Ip], c);
          c = mma16(al, dah[Ip], c);
          c = mma16(ah, dal[Ip], c);
          if (Ip == I) ad = c;
          else ao += ld4(&sm.Fe[Ip][I][kc]) * c;
        }
      }
      f32x4 pp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 vv = from_bits<bf16x8>(tile_row8(sm.v, row, 32 * ks + 8 * gq));
        pp = mma32(from_bits<bf16x8>(tile_row8(sm.dh[0], 16 * kt + r, 32 * ks + 8 * gq)), vv, pp);
        pp = mma32(from_bits<bf16x8>(tile_row8(sm.dh[1], 16 * kt + r, 32 * ks + 8 * gq)), vv, pp);
      }
      const f32x4 G4 = ld4(&sm.G[row][kc]), M4 = ld4(&sm.M[I][kc]), E4 = ld4(&sm.E[I][kc]);
      const f32x4 g4 = ld4(&sm.gam[kc]);
      f32x4 dki, dks;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dki[i] = scale * fmaf(cexp2(M4[i] - G4[i]), ad[i], cexp2(E4[i] - G4[i]) * ao[i]);
        dks[i] = cexp2(g4[i] - G4[i]) * pp[i];
      }
      const f32x4 kf = widen4(tile_row4(sm.k, row, kc));
      dGv[u] -= kf * dki;
      tdk[u] = kf * dks;
      if (row_ok) *reinterpret_cast<uint2 *>(dk + orow * KD + kc) = pack4(dki + dks);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // ---- (7) dv: A blocks (t in I' >= I, s in I), then per value tile
  {
    f32x8 kmf[2], kef[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int cc = 32 * ks + 8 * gq;
      kmf[ks] = widen8(tile_row8(sm.km[0], row, cc)) + widen8(tile_row8(sm.km[1], row, cc));
      kef[ks] = widen8(tile_row8(sm.ke[0], row, cc)) + widen8(tile_row8(sm.ke[1], row, cc));
    }
    s16x4 aah[4], aal[4];
#pragma unroll
    for (int Ip = 0; Ip < 4; ++Ip) {
      if (Ip >= I) {
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int cc = 32 * ks + 8 * gq;
          f32x8 b = kmf[ks];
          if (Ip != I) {
            const f32x4 f0 = ld4(&sm.Fe[Ip][I][cc]), f1 = ld4(&sm.Fe[Ip][I][cc + 4]);
            b = kef[ks] * f32x8{f0[0], f0[1], f0[2], f0[3], f1[0], f1[1], f1[2], f1[3]};
          }
          bf16x8 bh, bl;
          split8(b, bh, bl);
          const bf16x8 qh = from_bits<bf16x8>(tile_row8(sm.qm[0], 16 * Ip + r, cc));
          const bf16x8 ql = from_bits<bf16x8>(tile_row8(sm.qm[1], 16 * Ip + r, cc));
          c = mma32(qh, bh, c);
          c = mma32(ql, bh, c);
          c = mma32(qh, bl, c);
        }
        c *= scale;
        if (Ip == I) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (r > 4 * gq + i) c[i] = 0.f;   // s > t
        }
        split4(c, aah[Ip], aal[Ip]);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int vt = 2 * P + u, vc = 16 * vt + 4 * gq;
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int Ip = 0; Ip < 4; ++Ip) {
        if (Ip >= I) {
          const s16x4 a = tr_read4(sm.dout, 16 * Ip + 4 * gq, 16 * vt, lane);
          c = mma16(a, aah[Ip], c);
          c = mma16(a, aal[Ip], c);
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int ra = 32 * ks + 8 * gq;
        const bf16x8 ah = tr_operand<bf16x8>(sm.dh[0], ra, ra + 4, 16 * vt, lane);
        const bf16x8 al = tr_operand<bf16x8>(sm.dh[1], ra, ra + 4, 16 * vt, lane);
        const bf16x8 bh = from_bits<bf16x8>(tile_row8(sm.kb[0], row, ra));
        const bf16x8 bl = from_bits<bf16x8>(tile_row8(sm.kb[1], row, ra));
        c = mma32(ah, bh, c);
        c = mma32(al, bh, c);
        c = mma32(ah, bl, c);
      }
      if (row_ok && vc < V) *reinterpret_cast<uint2 *>(dv + orow * V + vc) = pack4(c);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // ---- (8) h <- 2^gamma h + (k 2^(gamma - G))^T v for keys 16 I .., value tiles 2P, 2P + 1
  {
    const f32x4 d4 = ld4(&sm.dgam[16 * I + 4 * gq]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int vt = 2 * P + u;
      hs[u] *= d4;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int ra = 32 * ks + 8 * gq;
        const bf16x8 ah = tr_operand<bf16x8>(sm.kb[0], ra, ra + 4, 16 * I, lane);
        const bf16x8 al = tr_operand<bf16x8>(sm.kb[1], ra, ra + 4, 16 * I, lane);
        const bf16x8 b = tr_operand<bf16x8>(sm.v, ra, ra + 4, 16 * vt, lane);
        hs[u] = mma32(ah, b, hs[u]);
        hs[u] = mma32(al, b, hs[u]);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // ---- (9) dg_t = 2^gamma sum_v h dh + sum_{j < t} tdk_j + sum_{r >= t} dG_r
  // (dG = q dq - k dk without the state term of dk, whose share tdk of the
  // chunk-total decay's gradient it would cancel)
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x = dGv[u][i];   // suffix sums over the block's rows (r)
      x += row_shl<1>(x);
      x += row_shl<2>(x);
      x += row_shl<4>(x);
      x += row_shl<8>(x);
      dGv[u][i] = x;
      tdk[u][i] = row_inclusive_scan(tdk[u][i]);
    }
    const int kc = 16 * (2 * P + u) + 4 * gq;
    if (r == 0) *reinterpret_cast<f32x4 *>(&sm.btot[0][I][kc]) = dGv[u];
    if (r == 15) *reinterpret_cast<f32x4 *>(&sm.btot[1][I][kc]) = tdk[u];
  }
  lds_barrier();
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int kc = 16 * (2 * P + u) + 4 * gq;
    f32x4 out = ld4(&sm.dgam[kc]) * ld4(&sm.hdh[kc]);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (b < I) out += ld4(&sm.btot[1][b][kc]);
      if (b > I) out += ld4(&sm.btot[0][b][kc]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] += dGv[u][i] + row_shr<1>(tdk[u][i]);
    if (row_ok) {
      if constexpr (GF32) *reinterpret_cast<f32x4 *>(static_cast<float *>(dg) + orow * KD + kc) = out;
      else *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(dg) + orow * KD + kc) = pack4(out);
    }
  }
}

template <bool GF32>
__global__ __launch_bounds__(64 * kWW) void bwd_walk_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const void *__restrict__ g, const uint16_t *__restrict__ dout, const int64_t *__restrict__ cu,
    const int64_t *__restrict__ coff, const int64_t *__restrict__ sgoff, int n_seq, int64_t T, int H, int V,
    float scale, const float *__restrict__ dloc, const float *__restrict__ drv, const float *__restrict__ sin_,
    const float *__restrict__ dsend, uint16_t *__restrict__ dq, uint16_t *__restrict__ dk, uint16_t *__restrict__ dv,
    void *__restrict__ dg) {
  __shared__ SmemW sm;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int r = lane & 15, gq = lane >> 4;
  const int I = w & 3, P = w >> 2;
  const int h = static_cast<int>(blockIdx.x % H);
  const int64_t sg = blockIdx.x / H;
  if (sg >= sgoff[n_seq]) return;   // workgroup-uniform
  const int n = find_seq(sgoff, n_seq, sg);
  int64_t bos, eos;
  seq_bounds(cu, n, T, bos, eos);
  const int64_t nc = (eos - bos + BT - 1) / BT;
  const int64_t j0 = (sg - sgoff[n]) * kSegC;   // first chunk of the segment in the sequence
  const int m = static_cast<int>(min(static_cast<int64_t>(kSegC), nc - j0));
  const int64_t c0 = coff[n] + j0;              // its global chunk index
  const int64_t KV = static_cast<int64_t>(KD) * V;

  // staging pieces: 16-bit tiles row pr, columns pc .. pc + 7; fp32 tiles
  // rows fr and fr + 32, columns fc .. fc + 3 (re-derived in every chunk
  // through an opaque zero, so that their addresses are not hoisted out of
  // the chunk loop and spilled)
  struct Pieces {
    int pr, pc, fr, fc;
  };
  auto pieces = [&]() {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    const int t = tid + z;
    return Pieces{t >> 3, 8 * (t & 7), t >> 4, 4 * (t & 15)};
  };
  const float *dse_s = dsend + (sg * H + h) * KV;
  f32x4 dse[2];
  {
    const Pieces pp = pieces();
#pragma unroll
    for (int u = 0; u < 2; ++u)
      dse[u] = pp.fc < V ? ld4(dse_s + static_cast<int64_t>(pp.fr + 32 * u) * V + pp.fc) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // the state: lane holds h[16 I + 4 gq + i][16 (2P + u) + r]
  f32x4 hs[2];
  {
    const float *s0 = sin_ + ((sg + n) * H + h) * KV;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int vc = 16 * (2 * P + u) + r;
#pragma unroll
      for (int i = 0; i < 4; ++i) hs[u][i] = vc < V ? s0[static_cast<int64_t>(16 * I + 4 * gq + i) * V + vc] : 0.f;
    }
  }

  uint4 pq, pk, pv, pdo, pg16;
  f32x4 pg[2], pdl[2];
  float pdr[2];
  // Loads go to clamped (always valid) addresses; rows past the chunk and
  // columns past V are zeroed when staged (a select right after a load
  // would make the compiler wait for it at once).
  auto fetch = [&](int jl, const Pieces &pp) {
    const int pr = pp.pr, pc = pp.pc, fr = pp.fr, fc = pp.fc;
    const int64_t t0 = bos + (j0 + jl) * BT;
    const int last = static_cast<int>(min(static_cast<int64_t>(BT), eos - t0)) - 1;
    const int64_t orq = (t0 + min(pr, last)) * H + h;
    const int64_t rq = orq * KD + pc, rv = orq * V + (pc < V ? pc : 0);
    pq = *reinterpret_cast<const uint4 *>(q + rq);
    pk = *reinterpret_cast<const uint4 *>(k + rq);
    pv = *reinterpret_cast<const uint4 *>(v + rv);
    pdo = *reinterpret_cast<const uint4 *>(dout + rv);
    if constexpr (GF32) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
        pg[u] = ld4(static_cast<const float *>(g) + ((t0 + min(fr + 32 * u, last)) * H + h) * KD + fc);
    } else {
      pg16 = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(g) + rq);
    }
    if (jl + 1 < m) {   // dh[c] = dloc[c + 1] + 2^drv[c + 1] dsend
      const int64_t cc = c0 + jl + 1;
      const int fcv = fc < V ? fc : 0;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int key = fr + 32 * u;
        pdl[u] = ld4(dloc + (cc * H + h) * KV + static_cast<int64_t>(key) * V + fcv);
        pdr[u] = drv[(cc * H + h) * KD + key];
      }
    } else {            // the segment's last chunk: dh[c] = dsend
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        pdl[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        pdr[u] = 0.f;
      }
    }
  };

  fetch(0, pieces());
  for (int jl = 0; jl < m; ++jl) {
    const int64_t t0 = bos + (j0 + jl) * BT;
    const int nrows = static_cast<int>(min(static_cast<int64_t>(BT), eos - t0));
    const Pieces pp = pieces();
    const int pr = pp.pr, pc = pp.pc, fr = pp.fr, fc = pp.fc;
    // ---- (1) raw tiles, g, dh and h into LDS; then the next chunk's loads
    const bool okr = pr < nrows;
    tile_store8(sm.q, pr, pc, keep4(pq, okr));
    tile_store8(sm.k, pr, pc, keep4(pk, okr));
    tile_store8(sm.v, pr, pc, keep4(pv, okr && pc < V));
    tile_store8(sm.dout, pr, pc, keep4(pdo, okr && pc < V));
    if constexpr (GF32) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
        *reinterpret_cast<f32x4 *>(&sm.G[fr + 32 * u][fc]) = keepf4(pg[u], fr + 32 * u < nrows);
    } else {
      const f32x8 gv = widen8(keep4(pg16, okr));
      *reinterpret_cast<f32x4 *>(&sm.G[pr][pc]) = f32x4{gv[0], gv[1], gv[2], gv[3]};
      *reinterpret_cast<f32x4 *>(&sm.G[pr][pc + 4]) = f32x4{gv[4], gv[5], gv[6], gv[7]};
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const f32x4 d = keepf4(pdl[u] + cexp2(pdr[u]) * dse[u], fc < V);
      s16x4 hi, lo;
      split4(d, hi, lo);
      tile_store4(sm.dh[0], fr + 32 * u, fc, __builtin_bit_cast(uint2, hi));
      tile_store4(sm.dh[1], fr + 32 * u, fc, __builtin_bit_cast(uint2, lo));
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      s16x4 hi, lo;
      split4(hs[u], hi, lo);
      const int vc = 16 * (2 * P + u) + r;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sm.h[0][swz(16 * I + 4 * gq + i, vc)] = static_cast<uint16_t>(hi[i]);
        sm.h[1][swz(16 * I + 4 * gq + i, vc)] = static_cast<uint16_t>(lo[i]);
      }
    }
    if (jl + 1 < m) fetch(jl + 1, pp);
    lds_barrier();

    // ---- (2) log2 cumsum of g per key: thread (key, 8-row group)
    {
      const int key = tid & 63, rg = tid >> 6;
      float run[8], s = 0.f;
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) {
        s += sm.G[8 * rg + rr][key];
        run[rr] = s;
      }
      sm.psum[rg][key] = s;
      lds_barrier();
      float off = 0.f;
      for (int b = 0; b < rg; ++b) off += sm.psum[b][key];
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) sm.G[8 * rg + rr][key] = (run[rr] + off) * kLog2e;
      if (rg == kWW - 1) sm.gam[key] = (s + off) * kLog2e;
    }
    lds_barrier();

    // ---- (3) block references, factors and sum_v h dh per key
    if (tid < 64) {
      const int key = tid;
      float ep = 0.f, Mb[4], Eb[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        Eb[b] = sm.G[16 * b + 15][key];
        Mb[b] = 0.5f * (ep + Eb[b]);
        ep = Eb[b];
        sm.E[b][key] = Eb[b];
        sm.M[b][key] = Mb[b];
      }
#pragma unroll
      for (int a = 1; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < a; ++b) sm.Fe[a][b][key] = cexp2(Mb[a] - Eb[b]);
      sm.dgam[key] = cexp2(sm.gam[key]);
    }
    {
      const int key = tid >> 3, c8 = 8 * (tid & 7);
      const f32x8 hv = widen8(tile_row8(sm.h[0], key, c8)) + widen8(tile_row8(sm.h[1], key, c8));
      const f32x8 dv8 = widen8(tile_row8(sm.dh[0], key, c8)) + widen8(tile_row8(sm.dh[1], key, c8));
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) s = fmaf(hv[e], dv8[e], s);
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 4);
      if ((tid & 7) == 0) sm.hdh[key] = s;
    }
    lds_barrier();

    // ---- (4) decay-scaled operand tiles: piece (row pr, keys pc .. pc + 7)
    {
      const int B = pr >> 4;
      const f32x8 qf = widen8(tile_row8(sm.q, pr, pc)), kf = widen8(tile_row8(sm.k, pr, pc));
      f32x8 Gv, Mv, Ev, gv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        Gv[e] = sm.G[pr][pc + e];
        Mv[e] = sm.M[B][pc + e];
        Ev[e] = sm.E[B][pc + e];
        gv[e] = sm.gam[pc + e];
      }
      f32x8 xq, xm, xe, xb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = Gv[e] - Mv[e];
        xq[e] = qf[e] * cexp2(x);
        xm[e] = kf[e] * cexp2(-x);
        xe[e] = kf[e] * cexp2(Ev[e] - Gv[e]);
        xb[e] = kf[e] * cexp2(gv[e] - Gv[e]);
      }
      bf16x8 hi, lo;
      split8(xq, hi, lo);
      tile_store8(sm.qm[0], pr, pc, to_bits(hi));
      tile_store8(sm.qm[1], pr, pc, to_bits(lo));
      split8(xm, hi, lo);
      tile_store8(sm.km[0], pr, pc, to_bits(hi));
      tile_store8(sm.km[1], pr, pc, to_bits(lo));
      split8(xe, hi, lo);
      tile_store8(sm.ke[0], pr, pc, to_bits(hi));
      tile_store8(sm.ke[1], pr, pc, to_bits(lo));
      split8(xb, hi, lo);
      tile_store8(sm.kb[0], pr, pc, to_bits(hi));
      tile_store8(sm.kb[1], pr, pc, to_bits(lo));
    }
    lds_barrier();

    if (P == 0) walk_chunk<GF32, 0>(sm, I, lane, nrows, t0, H, h, V, scale, hs, dq, dk, dv, dg);
    else walk_chunk<GF32, 1>(sm, I, lane, nrows, t0, H, h, V, scale, hs, dq, dk, dv, dg);
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
  // bf16: the walking chunk pass carries the forward state, so the forward
  // local pass keeps only its segment end states
  constexpr bool kWalk = DT == SSLA_BF16;
  if constexpr (kWalk)
    hipLaunchKernelGGL((bwd_seg_passes_tiles<GF32>), dim3(static_cast<unsigned>(2 * nb)), dim3(256), 0, st, Kp, Vp, Q,
                       DO, g, cu, w.coff, w.sgoff, n_seq, T, H, V, scale, nb, w.eloc, w.dtot, w.dloc, w.drv);
  else
    hipLaunchKernelGGL((bwd_seg_passes<DT, GF32>), dim3(static_cast<unsigned>(2 * nb)), dim3(256), 0, st, Kp, Vp, Q,
                       DO, g, cu, w.coff, w.sgoff, n_seq, T, H, V, scale, nb, w.hloc, w.dfw, w.eloc, w.dtot, w.dloc,
                       w.drv);
  const int64_t fold_threads = static_cast<int64_t>(n_seq) * H * KD * V;
  hipLaunchKernelGGL(bwd_fold_kernel, dim3(static_cast<unsigned>((fold_threads + 255) / 256)), dim3(256), 0, st,
                     w.coff, w.sgoff, n_seq, H, V, h0, dht, w.eloc, w.dtot, w.dloc, w.sin_, w.dsend, dh0);
  if constexpr (kWalk) {
    hipLaunchKernelGGL((bwd_walk_kernel<GF32>), dim3(static_cast<unsigned>(nb)), dim3(64 * kWW), 0, st, Q, Kp, Vp, g,
                       DO, cu, w.coff, w.sgoff, n_seq, T, H, V, scale, w.dloc, w.drv, w.sin_, w.dsend,
                       static_cast<uint16_t *>(dq), static_cast<uint16_t *>(dk), static_cast<uint16_t *>(dv), dg);
  } else {
    hipLaunchKernelGGL((bwd_chunk_kernel<DT, GF32>), dim3(static_cast<unsigned>(cmax * H)), dim3(64 * kCW), 0, st, Q,
                       Kp, Vp, g, DO, cu, w.coff, w.sgoff, n_seq, T, H, V, scale, w.hloc, w.dfw, w.dloc, w.drv,
                       w.sin_, w.dsend, static_cast<uint16_t *>(dq), static_cast<uint16_t *>(dk),
                       static_cast<uint16_t *>(dv), dg);
  }
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
