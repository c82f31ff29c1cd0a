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
// as split bf16 triples (see mma3) with fp32 accumulation; states, A, dA and
// dg are fp32.
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
typedef float f32x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4 mma3(const float (&a)[8], const float (&b)[8], f32x4 c) {
  const f32x8 va = {a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7]};
  const f32x8 vb = {b[0], b[1], b[2], b[3], b[4], b[5], b[6], b[7]};
  const bf16x8 ah = __builtin_convertvector(va, bf16x8), bh = __builtin_convertvector(vb, bf16x8);
  const bf16x8 al = __builtin_convertvector(va - __builtin_convertvector(ah, f32x8), bf16x8);
  const bf16x8 bl = __builtin_convertvector(vb - __builtin_convertvector(bh, f32x8), bf16x8);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
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

// coff[n] = chunks of sequences 0..n-1 (coff[n_seq] = all chunks).  One
// workgroup; sequence n's state slots are coff[n] + n .. coff[n+1] + n.
__global__ __launch_bounds__(256) void bwd_offsets_kernel(const int64_t *__restrict__ cu, int n_seq, int64_t T,
                                                          int64_t *__restrict__ coff) {
  __shared__ int64_t part[256];
  int64_t carry = 0;
  for (int base = 0; base < n_seq; base += 256) {
    const int n = base + static_cast<int>(threadIdx.x);
    int64_t c = 0;
    if (n < n_seq) {
      int64_t bos, eos;
      seq_bounds(cu, n, T, bos, eos);
      c = (eos - bos + BT - 1) / BT;
    }
    part[threadIdx.x] = c;
    __syncthreads();
    for (int d = 1; d < 256; d <<= 1) {   // inclusive scan (Hillis-Steele)
      const int64_t x = threadIdx.x >= static_cast<unsigned>(d) ? part[threadIdx.x - d] : 0;
      __syncthreads();
      part[threadIdx.x] += x;
      __syncthreads();
    }
    if (n < n_seq) coff[n] = carry + part[threadIdx.x] - c;
    carry += part[255];
    __syncthreads();
  }
  if (threadIdx.x == 0) coff[n_seq] = carry;
}

// --------------------------------------------------------- state passes --
// One wavefront per (sequence, head, 16 value columns v0..v0+15).  Lane l
// holds state rows (keys) 16 Kb + 4 (l / 16) + i of tile Kb, column l % 16.
// REV = false: X = k, Y = v, factor e^(G_last - G_t), chunks in order, the
//              state is stored before each chunk and after the last one.
// REV = true : X = scale q, Y = do, factor e^(G_t), chunks in reverse, the
//              gradient is stored after the end (dht) and after each chunk.
template <bool REV, int DT, bool GF32>
__global__ __launch_bounds__(64) void bwd_state_pass(const uint16_t *__restrict__ X, const uint16_t *__restrict__ Y,
                                                     const void *__restrict__ g, const int64_t *__restrict__ cu,
                                                     const int64_t *__restrict__ coff, int n_seq, int64_t T, int H,
                                                     int V, float xscale, const float *__restrict__ s_init,
                                                     float *__restrict__ slots, float *__restrict__ s_out) {
  __shared__ uint16_t xs[BT][KD];
  __shared__ float gs[BT][KD];
  __shared__ uint16_t ys[BT][16];
  __shared__ float glast[KD];
  const int lane = threadIdx.x;
  const int nvb = V / 16;
  const int64_t item = blockIdx.x;
  const int vb = static_cast<int>(item % nvb);
  const int h = static_cast<int>((item / nvb) % H);
  const int n = static_cast<int>(item / (static_cast<int64_t>(nvb) * H));
  if (n >= n_seq) return;
  const int v0 = vb * 16;
  int64_t bos, eos;
  seq_bounds(cu, n, T, bos, eos);
  const int64_t nc = (eos - bos + BT - 1) / BT;
  const int64_t slot0 = coff[n] + n;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t KV = static_cast<int64_t>(KD) * V;
  auto sidx = [&](int64_t slot, int key) { return (slot * H + h) * KV + static_cast<int64_t>(key) * V + v0 + col; };

  f32x4 acc[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kb * 16 + grp * 4 + i;
      acc[kb][i] = s_init ? s_init[((static_cast<int64_t>(n) * H + h) * KD + key) * V + v0 + col] : 0.f;
    }
  auto store = [&](int64_t slot) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) slots[sidx(slot, kb * 16 + grp * 4 + i)] = acc[kb][i];
  };
  if (REV) store(slot0 + nc);

  for (int64_t jj = 0; jj < nc; ++jj) {
    const int64_t j = REV ? nc - 1 - jj : jj;
    if (!REV) store(slot0 + j);
    const int64_t t0 = bos + j * BT;
    const int nrows = static_cast<int>(min(static_cast<int64_t>(BT), eos - t0));
    // stage: lane = key for X and the gate cumsum; Y 16 columns
    float run = 0.f;
#pragma unroll 8
    for (int r = 0; r < BT; ++r) {
      const bool ok = r < nrows;
      const int64_t row = (t0 + r) * H + h;
      xs[r][lane] = ok ? X[row * KD + lane] : static_cast<uint16_t>(0);
      run += ok ? load_g<GF32, DT>(g, row * KD + lane) * kLog2e : 0.f;
      gs[r][lane] = run;
    }
    glast[lane] = run;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const int r = rr * 4 + grp;
      ys[r][col] = r < nrows ? Y[((t0 + r) * H + h) * V + v0 + col] : static_cast<uint16_t>(0);
    }
    __syncthreads();
    // decay, then add X~^T Y (keys x time) x (time x 16 columns)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[kb][i] *= cexp2(glast[kb * 16 + grp * 4 + i]);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        float a[8], b[8];
        const int key = kb * 16 + col;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int t = ks * 32 + grp * 8 + e;
          const float x = Elt<DT>::f(xs[t][key]) * xscale;
          a[e] = x * cexp2(REV ? gs[t][key] : glast[key] - gs[t][key]);
          b[e] = Elt<DT>::f(ys[t][col]);
        }
        acc[kb] = mma3(a, b, acc[kb]);
      }
    }
    __syncthreads();
    if (REV) store(slot0 + j);
  }
  if (!REV) store(slot0 + nc);
  if (REV && s_out) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        s_out[((static_cast<int64_t>(n) * H + h) * KD + kb * 16 + grp * 4 + i) * V + v0 + col] = acc[kb][i];
  }
}

// ------------------------------------------------------------ chunk pass --
// One workgroup (4 wavefronts) per (chunk, head).  Wavefront I owns rows
// 16 I .. 16 I + 15: it computes those rows of A and dA, then dq, dk, dv and
// the q dq - k dk terms of those rows; dg is a reverse cumsum over the
// chunk.  q, k, v, do are staged as rows of 64 input-dtype values (value
// columns padded with zeros to VP = V rounded up to 32).
struct __align__(16) SmemC {
  uint16_t q[BT][KD], k[BT][KD], v[BT][64], dout[BT][64];
  float dh[KD][64];    // dh[c] as [key][value]
  union {
    struct {
      float A[BT][BT], dA[BT][BT];
    } p;
    float r[BT][KD];   // q dq - k dk (after the products)
  } u;
  float G[BT][KD];     // log2 cumsum
  float M[4][KD];      // block reference points
  float glast[KD];
  float term[KD];      // sum_v dh[c] h[c+1]
  float bsum[4][KD];
};

template <int DT, bool GF32>
__global__ __launch_bounds__(256) void bwd_chunk_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const void *__restrict__ g, const uint16_t *__restrict__ dout, const int64_t *__restrict__ cu,
    const int64_t *__restrict__ coff, int n_seq, int64_t T, int H, int V, float scale,
    const float *__restrict__ hs, const float *__restrict__ dhs, uint16_t *__restrict__ dq,
    uint16_t *__restrict__ dk, uint16_t *__restrict__ dv, void *__restrict__ dg) {
  __shared__ SmemC sm;
  auto X = [](uint16_t b) { return Elt<DT>::f(b); };   // a staged input value
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int h = static_cast<int>(blockIdx.x % H);
  const int64_t c = blockIdx.x / H;
  if (c >= coff[n_seq]) return;   // workgroup-uniform
  // sequence of chunk c: the last n with coff[n] <= c
  int lo = 0, hi = n_seq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (coff[mid] <= c) lo = mid;
    else hi = mid - 1;
  }
  const int n = lo;
  int64_t bos, eos;
  seq_bounds(cu, n, T, bos, eos);
  const int64_t j = c - coff[n];
  const int64_t t0 = bos + j * BT;
  const int nrows = static_cast<int>(min(static_cast<int64_t>(BT), eos - t0));
  const int64_t slot = coff[n] + n + j;   // h[c] entering, slot + 1: leaving state / dh[c]
  const int64_t KV = static_cast<int64_t>(KD) * V;
  const float *hc = hs + (slot * H + h) * KV;
  const float *hn = hs + ((slot + 1) * H + h) * KV;
  const float *dhc = dhs + ((slot + 1) * H + h) * KV;
  const int VP = (V + 31) & ~31;

  // ---- staging: q, k, v, do rows (4 threads per row, 16 columns each)
  {
    const int r = tid >> 2, c0 = (tid & 3) * 16;
    const bool ok = r < nrows;
    const int64_t row = (t0 + r) * H + h;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      sm.q[r][c0 + e] = ok ? q[row * KD + c0 + e] : static_cast<uint16_t>(0);
      sm.k[r][c0 + e] = ok ? k[row * KD + c0 + e] : static_cast<uint16_t>(0);
      const bool okv = ok && c0 + e < V;
      sm.v[r][c0 + e] = okv ? v[row * V + c0 + e] : static_cast<uint16_t>(0);
      sm.dout[r][c0 + e] = okv ? dout[row * V + c0 + e] : static_cast<uint16_t>(0);
      sm.dh[r][c0 + e] = c0 + e < V ? dhc[static_cast<int64_t>(r) * V + c0 + e] : 0.f;   // row r = key
    }
  }
  if (w == 0) {   // gate cumsum per key (lane = key), block reference points
    float run = 0.f;
#pragma unroll 8
    for (int r = 0; r < BT; ++r) {
      run += r < nrows ? load_g<GF32, DT>(g, ((t0 + r) * H + h) * KD + lane) * kLog2e : 0.f;
      sm.G[r][lane] = run;
    }
    sm.glast[lane] = run;
    float ep = 0.f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float eb = sm.G[b * 16 + 15][lane];
      sm.M[b][lane] = 0.5f * (ep + eb);
      ep = eb;
    }
  } else if (w == 1) {   // sum_v dh[c] * (state leaving the chunk)
    float s = 0.f;
    for (int vv = 0; vv < V; ++vv) s += dhc[static_cast<int64_t>(lane) * V + vv] * hn[static_cast<int64_t>(lane) * V + vv];
    sm.term[lane] = s;
  }
  __syncthreads();

  const int I = w;   // this wavefront's row block
  // ---- A and dA, rows of block I (zero above the diagonal)
  for (int J = 0; J < 4; ++J) {
    f32x4 a4 = {0.f, 0.f, 0.f, 0.f}, d4 = {0.f, 0.f, 0.f, 0.f};
    if (J <= I) {
      const int t = 16 * I + col, s = 16 * J + col;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        float a[8], b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int kk = ks * 32 + grp * 8 + e;
          const float m = sm.M[I][kk];
          a[e] = X(sm.q[t][kk]) * cexp2(sm.G[t][kk] - m);
          b[e] = X(sm.k[s][kk]) * cexp2(m - sm.G[s][kk]);
        }
        a4 = mma3(a, b, a4);
      }
      for (int vs = 0; vs < VP; vs += 32) {
        float a[8], b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int vc = vs + grp * 8 + e;
          a[e] = X(sm.dout[t][vc]);
          b[e] = X(sm.v[s][vc]);
        }
        d4 = mma3(a, b, d4);
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
  __syncthreads();

  // ---- dq (rows t of block I), keys in 4 tiles
  float dqv[4][4], dkv[4][4];
  {
    f32x4 ai[4], ae[4];
#pragma unroll
    for (int N = 0; N < 4; ++N) {
      ai[N] = f32x4{0.f, 0.f, 0.f, 0.f};
      ae[N] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int t = 16 * I + col;
    const int s_end = 16 * (I + 1);
    for (int ss = 0; ss < s_end; ss += 32) {   // intra: dA[t, s] (k e^(M_I - G))[s, key]
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = (sm.u.p.dA[t][ss + grp * 8 + e]);
#pragma unroll
      for (int N = 0; N < 4; ++N) {
        const int key = N * 16 + col;
        const float m = sm.M[I][key];
        float b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int s = ss + grp * 8 + e;
          b[e] = s < s_end ? X(sm.k[s][key]) * cexp2(m - sm.G[s][key]) : 0.f;
        }
        ai[N] = mma3(a, b, ai[N]);
      }
    }
    for (int vs = 0; vs < VP; vs += 32) {   // inter: do[t, v] h[c][key, v]
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = X(sm.dout[t][vs + grp * 8 + e]);
#pragma unroll
      for (int N = 0; N < 4; ++N) {
        const int key = N * 16 + col;
        float b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int vc = vs + grp * 8 + e;
          b[e] = vc < V ? hc[static_cast<int64_t>(key) * V + vc] : 0.f;
        }
        ae[N] = mma3(a, b, ae[N]);
      }
    }
#pragma unroll
    for (int N = 0; N < 4; ++N)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tt = 16 * I + grp * 4 + i, key = N * 16 + col;
        const float gt = sm.G[tt][key];
        dqv[N][i] = ai[N][i] * cexp2(gt - sm.M[I][key]) + scale * ae[N][i] * cexp2(gt);
      }
  }
  // ---- dk (rows s of block I)
  {
    f32x4 ai[4], ae[4];
#pragma unroll
    for (int N = 0; N < 4; ++N) {
      ai[N] = f32x4{0.f, 0.f, 0.f, 0.f};
      ae[N] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int s = 16 * I + col;
    const int t_beg = 16 * I;
    for (int ts = t_beg & ~31; ts < BT; ts += 32) {   // intra: dA[t, s] (q e^(G - M_I))[t, key]
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = (sm.u.p.dA[ts + grp * 8 + e][s]);
#pragma unroll
      for (int N = 0; N < 4; ++N) {
        const int key = N * 16 + col;
        const float m = sm.M[I][key];
        float b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int t = ts + grp * 8 + e;
          b[e] = t >= t_beg ? X(sm.q[t][key]) * cexp2(sm.G[t][key] - m) : 0.f;
        }
        ai[N] = mma3(a, b, ai[N]);
      }
    }
    for (int vs = 0; vs < VP; vs += 32) {   // inter: v[s, v] dh[c][key, v]
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = X(sm.v[s][vs + grp * 8 + e]);
#pragma unroll
      for (int N = 0; N < 4; ++N) {
        const int key = N * 16 + col;
        float b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) b[e] = (sm.dh[key][vs + grp * 8 + e]);
        ae[N] = mma3(a, b, ae[N]);
      }
    }
#pragma unroll
    for (int N = 0; N < 4; ++N)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ss = 16 * I + grp * 4 + i, key = N * 16 + col;
        const float gs = sm.G[ss][key];
        dkv[N][i] = ai[N][i] * cexp2(sm.M[I][key] - gs) + ae[N][i] * cexp2(sm.glast[key] - gs);
      }
  }
  // ---- dv (rows s of block I), value columns in tiles of 16
  for (int N = 0; N < VP / 16; ++N) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int s = 16 * I + col;
    const int vc = N * 16 + col;
    const int t_beg = 16 * I;
    for (int ts = t_beg & ~31; ts < BT; ts += 32) {   // intra: A[t, s] do[t, v]
      float a[8], b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = ts + grp * 8 + e;
        a[e] = (sm.u.p.A[t][s]);
        b[e] = X(sm.dout[t][vc]);
      }
      acc = mma3(a, b, acc);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {   // inter: (k e^(G_last - G))[s, key] dh[c][key, v]
      float a[8], b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kk = ks * 32 + grp * 8 + e;
        a[e] = X(sm.k[s][kk]) * cexp2(sm.glast[kk] - sm.G[s][kk]);
        b[e] = (sm.dh[kk][vc]);
      }
      acc = mma3(a, b, acc);
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
  for (int N = 0; N < 4; ++N)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tt = 16 * I + grp * 4 + i, key = N * 16 + col;
      sm.u.r[tt][key] = X(sm.q[tt][key]) * dqv[N][i] - X(sm.k[tt][key]) * dkv[N][i];
      if (tt < nrows) {
        const int64_t o = ((t0 + tt) * H + h) * KD + key;
        dq[o] = Elt<DT>::b(dqv[N][i]);
        dk[o] = Elt<DT>::b(dkv[N][i]);
      }
    }
  __syncthreads();
  // ---- dg: reverse cumsum over the chunk + the leaving-state term;
  // thread (w, lane): key = lane, rows 16 w .. 16 w + 15
  {
    const int key = lane;
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += sm.u.r[16 * w + r][key];
    sm.bsum[w][key] = s;
    __syncthreads();
    float run = sm.term[key];
    for (int b = 3; b > w; --b) run += sm.bsum[b][key];
#pragma unroll
    for (int r = 15; r >= 0; --r) {
      const int tt = 16 * w + r;
      run += sm.u.r[tt][key];
      if (tt < nrows) {
        const int64_t o = ((t0 + tt) * H + h) * KD + key;
        if constexpr (GF32) static_cast<float *>(dg)[o] = run;
        else static_cast<uint16_t *>(dg)[o] = Elt<DT>::b(run);
      }
    }
  }
}

template <int DT, bool GF32>
int launch_bwd(const void *q, const void *k, const void *v, const void *g, const int64_t *cu, int n_seq, int64_t T,
               int H, int V, float scale, const float *h0, const void *dout, const float *dht, void *dq, void *dk,
               void *dv, void *dg, float *dh0, int64_t *coff, float *hs, float *dhs, hipStream_t st) {
  const auto *Q = static_cast<const uint16_t *>(q);
  const auto *Kp = static_cast<const uint16_t *>(k);
  const auto *Vp = static_cast<const uint16_t *>(v);
  const auto *DO = static_cast<const uint16_t *>(dout);
  hipLaunchKernelGGL(bwd_offsets_kernel, dim3(1), dim3(256), 0, st, cu, n_seq, T, coff);
  const int64_t passes = static_cast<int64_t>(n_seq) * H * (V / 16);
  hipLaunchKernelGGL((bwd_state_pass<false, DT, GF32>), dim3(static_cast<unsigned>(passes)), dim3(64), 0, st, Kp, Vp, g,
                     cu, coff, n_seq, T, H, V, 1.f, h0, hs, static_cast<float *>(nullptr));
  hipLaunchKernelGGL((bwd_state_pass<true, DT, GF32>), dim3(static_cast<unsigned>(passes)), dim3(64), 0, st, Q, DO, g,
                     cu, coff, n_seq, T, H, V, scale, dht, dhs, dh0);
  const int64_t chunks = (T + BT - 1) / BT + n_seq;
  hipLaunchKernelGGL((bwd_chunk_kernel<DT, GF32>), dim3(static_cast<unsigned>(chunks * H)), dim3(256), 0, st, Q, Kp, Vp,
                     g, DO, cu, coff, n_seq, T, H, V, scale, hs, dhs, static_cast<uint16_t *>(dq),
                     static_cast<uint16_t *>(dk), static_cast<uint16_t *>(dv), dg);
  return launch_status("gla_chunk_bwd");
}

inline int64_t bwd_slots(int n_seq, int64_t T) { return (T + BT - 1) / BT + 2 * static_cast<int64_t>(n_seq); }
inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

}  // namespace
}  // namespace ssla

extern "C" size_t ssla_gla_chunk_bwd_workspace_size(int n_seq, int64_t T, int H, int K, int V) {
  if (n_seq < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0) return 0;
  const size_t st = static_cast<size_t>(ssla::bwd_slots(n_seq, T)) * H * K * V * sizeof(float);
  return ssla::align256(sizeof(int64_t) * (n_seq + 1)) + 2 * ssla::align256(st);
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
  if (n_seq == 0 || T == 0) return SSLA_OK;
  SSLA_CHECK_ARG(q && k && v && g && cu_seqlens && dout && dq && dk && dv && dg, "gla_chunk_bwd: null pointer");
  const size_t need = ssla_gla_chunk_bwd_workspace_size(n_seq, T, H, K, V);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("gla_chunk_bwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  SSLA_CHECK_ARG(aligned(workspace, 16), "gla_chunk_bwd: workspace must be 16-byte aligned");
  const int64_t chunks = (T + BT - 1) / BT + n_seq;
  if (chunks * H > 0x7fffffff || static_cast<int64_t>(n_seq) * H * (V / 16) > 0x7fffffff) {
    set_error("gla_chunk_bwd: too many chunks");
    return SSLA_ERR_UNSUPPORTED;
  }
  char *base = static_cast<char *>(workspace);
  int64_t *coff = reinterpret_cast<int64_t *>(base);
  const size_t st_bytes = align256(static_cast<size_t>(bwd_slots(n_seq, T)) * H * K * V * sizeof(float));
  float *hs = reinterpret_cast<float *>(base + align256(sizeof(int64_t) * (n_seq + 1)));
  float *dhs = reinterpret_cast<float *>(reinterpret_cast<char *>(hs) + st_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool gf32 = g_dtype == SSLA_F32;
  if (dtype == SSLA_BF16)
    return gf32 ? launch_bwd<SSLA_BF16, true>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, dout, dht, dq, dk,
                                              dv, dg, dh0, coff, hs, dhs, st)
                : launch_bwd<SSLA_BF16, false>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, dout, dht, dq,
                                               dk, dv, dg, dh0, coff, hs, dhs, st);
  return gf32 ? launch_bwd<SSLA_F16, true>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, dout, dht, dq, dk, dv,
                                           dg, dh0, coff, hs, dhs, st)
              : launch_bwd<SSLA_F16, false>(q, k, v, g, cu_seqlens, n_seq, T, H, V, scale, h0, dout, dht, dq, dk,
                                            dv, dg, dh0, coff, hs, dhs, st);
}
