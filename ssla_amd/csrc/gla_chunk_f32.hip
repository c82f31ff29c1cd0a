// Chunked GLA in fp32: forward and backward for fp32 q, k, v, g (the
// reference runs its chunk pipeline for fp32 inputs too: ops/gla/chunk.py
// 906-960 forward, 963-1053 backward, with TF32 operands in most of its
// dots; here every product is fp32).
//
// Chunks of 64 rows restart at every sequence start; G is the chunk-local
// inclusive cumsum of g (log2-scaled), gamma = G at the chunk's last row,
// s = scale:
//   A_ij = s sum_k q_ik k_jk 2^(G_ik - G_jk)  (j <= i)
//   o    = s (q 2^G) S_c + A v
//   S_c+1 = 2^gamma S_c + (k 2^(gamma - G))^T v
// Every decay factor is kept at or below 1, so the exponent clamp at -126
// (v_exp_f32 range) only ever replaces a value that is itself below 2^-126:
// * diagonal 16-row blocks (j, i in one block, j <= i): 2^(G_i - G_j)
//   directly, one exponential of a non-positive argument per term;
// * blocks J < I: 2^(G_i - G_j) = 2^(G_i - E_J) 2^(E_J - G_j) with E_J = G at
//   the last row of block J (both factors <= 1): k~_j = k_j 2^(E_J - G_j)
//   per row, and the q side per (row, J) -- A and dq; or
//   2^(G_i - S_I) 2^(S_I - G_j) with S_I = G at the first row of block I:
//   q~_i = q_i 2^(G_i - S_I) per row, and the k side per (row, I) -- dk;
// * o, the state and dh use 2^G and 2^(gamma - G) (<= 1) directly.
// All arithmetic is fp32 on the VALU: the matrix cores' fp32 rate is only
// twice the VALU's, and these kernels serve the fp32 (training and
// reference-precision) path, where the bf16 kernels do not apply.
//
// Forward: one workgroup per (sequence, head, 16-column V tile) walks the
// sequence's chunks with its state tile in LDS.  Backward: one workgroup per
// (sequence, head) (K, V <= 64) first walks forward storing each chunk's
// entering state in the workspace, then walks back: dv = A^T dO + k_d dh,
// dq, dk from dO h^T, v dh^T and dA = (dO v^T) masked, dg = reverse cumsum
// of dG = q dq - k dk plus the chunk-total decay's term, dh <- 2^gamma dh +
// s (q 2^G)^T dO.  dG is formed without the terms that cancel exactly (the
// j = i term of A, and the state term of dk against the same term of the
// chunk-total decay's gradient): with strongly decaying gates dg is small
// next to q dq and k dk, and those terms would leave only their rounding.
#include "common.h"

namespace ssla {
namespace {

constexpr int kC = 64;        // chunk rows
constexpr int kP = 65;        // LDS row pitch (floats): conflict-free column walks
constexpr int kVT = 16;       // value columns per forward workgroup
constexpr int kThreads = 256;

__device__ __forceinline__ float ex2c(float x) { return fast_exp2(fminf(fmaxf(x, -126.f), 126.f)); }

__device__ __forceinline__ void seq_bounds(const int64_t *cu, int n, int64_t T, int64_t &bos, int64_t &eos) {
  bos = min(max(cu[n], (int64_t)0), T);
  eos = min(max(cu[n + 1], bos), T);
}

// Per-key references of a chunk (64 threads, one key each, after the
// cumsum): E[J] = G at row 16 J + 15, S[I] = G at row 16 I, PE[J] =
// 2^(gamma - E[J]), DL = 2^gamma, GAM = gamma.
struct ChunkRefs {
  float E[4][64], S[4][64], PE[4][64], DL[64], GAM[64];
};

// Chunk-local cumsum of the gates (log2-scaled, in place) and the
// references; rows past the chunk hold g = 0, so G stays at gamma there.
__device__ __forceinline__ void chunk_cumsum(float (*sG)[kP], ChunkRefs &R) {
  const int kk = threadIdx.x;
  if (kk >= 64) return;
  float acc = 0.f;
  for (int r = 0; r < kC; ++r) {
    acc += sG[r][kk];
    sG[r][kk] = acc;
  }
#pragma unroll
  for (int I = 0; I < 4; ++I) {
    R.E[I][kk] = sG[16 * I + 15][kk];
    R.S[I][kk] = sG[16 * I][kk];
    R.PE[I][kk] = ex2c(acc - sG[16 * I + 15][kk]);
  }
  R.DL[kk] = ex2c(acc);
  R.GAM[kk] = acc;
}

// k~_j = k_j 2^(E_J - G_j) (into sKt) and, when sQt is given,
// q~_i = q_i 2^(G_i - S_I) (into sQt).
__device__ __forceinline__ void chunk_tilde(const float (*sQ)[kP], const float (*sK)[kP], const float (*sG)[kP],
                                            const ChunkRefs &R, float (*sKt)[kP], float (*sQt)[kP]) {
  for (int e = threadIdx.x; e < kC * 64; e += kThreads) {
    const int r = e >> 6, kk = e & 63, B = r >> 4;
    sKt[r][kk] = sK[r][kk] * ex2c(R.E[B][kk] - sG[r][kk]);
    if (sQt) sQt[r][kk] = sQ[r][kk] * ex2c(sG[r][kk] - R.S[B][kk]);
  }
}

// The 16 entries A_i,16J..16J+15 of thread (i, J), scale applied (zero
// above the diagonal): blocks J < I as (q_i 2^(G_i - E_J)) . k~_j, the
// diagonal block term by term.
__device__ __forceinline__ void a_row16(const float (*sQ)[kP], const float (*sK)[kP], const float (*sKt)[kP],
                                        const float (*sG)[kP], const ChunkRefs &R, int K, int i, int J, float scale,
                                        float (&a)[16]) {
  const int I = i >> 4;
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) a[jj] = 0.f;
  if (J > I) return;
  if (J < I) {
    for (int kk = 0; kk < K; ++kk) {
      const float qv = sQ[i][kk] * ex2c(sG[i][kk] - R.E[J][kk]);
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) a[jj] = fmaf(qv, sKt[16 * J + jj][kk], a[jj]);
    }
  } else {
    const int il = i - 16 * I;   // j = 16 I + jj <= i
    for (int kk = 0; kk < K; ++kk) {
      const float qv = sQ[i][kk], gi = sG[i][kk];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj)
        if (jj <= il) a[jj] = fmaf(qv * sK[16 * I + jj][kk], ex2c(gi - sG[16 * I + jj][kk]), a[jj]);
    }
  }
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) a[jj] *= scale;
}

// ---------------------------------------------------------------- forward --
__global__ __launch_bounds__(kThreads) void f32_fwd_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ g, const int64_t *__restrict__ cu, int n_seq, int64_t T, int H, int K, int V,
    float scale, const float *__restrict__ h0, float *__restrict__ o, float *__restrict__ ht) {
  __shared__ float sQ[kC][kP], sK[kC][kP], sKt[kC][kP], sG[kC][kP], sA[kC][kP];
  __shared__ float sV[kC][kVT], sS[64][kVT];
  __shared__ ChunkRefs R;
  const int tid = threadIdx.x;
  const int nvt = (V + kVT - 1) / kVT;
  const int64_t wg = blockIdx.x;
  const int vt = static_cast<int>(wg % nvt);
  const int h = static_cast<int>((wg / nvt) % H);
  const int n = static_cast<int>(wg / (static_cast<int64_t>(nvt) * H));
  const int v0 = vt * kVT;
  int64_t bos, eos;
  seq_bounds(cu, n, T, bos, eos);
  const int64_t sb = (static_cast<int64_t>(n) * H + h) * K * V;   // this (sequence, head)'s state
  for (int e = tid; e < 64 * kVT; e += kThreads) {
    const int kk = e / kVT, c = e % kVT;
    sS[kk][c] = (h0 && kk < K && v0 + c < V) ? h0[sb + static_cast<int64_t>(kk) * V + v0 + c] : 0.f;
  }
  const int ri = tid >> 2, q4 = tid & 3;   // row (or key) of this thread, and its quarter
  for (int64_t t0 = bos; t0 < eos; t0 += kC) {
    const int nc = static_cast<int>(min(static_cast<int64_t>(kC), eos - t0));
    __syncthreads();   // the previous chunk is done with the tiles
    for (int e = tid; e < kC * 64; e += kThreads) {
      const int r = e >> 6, kk = e & 63;
      const bool ok = r < nc && kk < K;
      const int64_t idx = ((t0 + r) * H + h) * K + kk;
      sQ[r][kk] = ok ? q[idx] : 0.f;
      sK[r][kk] = ok ? k[idx] : 0.f;
      sG[r][kk] = ok ? g[idx] * kLog2e : 0.f;
    }
    for (int e = tid; e < kC * kVT; e += kThreads) {
      const int r = e / kVT, c = e % kVT;
      sV[r][c] = (r < nc && v0 + c < V) ? v[((t0 + r) * H + h) * V + v0 + c] : 0.f;
    }
    __syncthreads();
    chunk_cumsum(sG, R);
    __syncthreads();
    chunk_tilde(sQ, sK, sG, R, sKt, nullptr);
    __syncthreads();
    {   // A, thread (row ri, block q4)
      float a[16];
      a_row16(sQ, sK, sKt, sG, R, K, ri, q4, scale, a);
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) sA[ri][16 * q4 + jj] = a[jj];
    }
    __syncthreads();
    {   // o: thread (row ri, columns 4 q4 .. 4 q4 + 3)
      const int c0 = 4 * q4;
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int kk = 0; kk < K; ++kk) {
        const float qg = sQ[ri][kk] * ex2c(sG[ri][kk]);   // q 2^G
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = fmaf(qg, sS[kk][c0 + c], acc[c]);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] *= scale;
      for (int j = 0; j <= ri; ++j) {
        const float aij = sA[ri][j];
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = fmaf(aij, sV[j][c0 + c], acc[c]);
      }
      if (ri < nc) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (v0 + c0 + c < V) o[((t0 + ri) * H + h) * V + v0 + c0 + c] = acc[c];
      }
    }
    __syncthreads();
    {   // S <- 2^gamma S + (k~ 2^(gamma - E_J))^T v: thread (key ri, columns 4 q4 ..)
      const int c0 = 4 * q4;
      float acc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = sS[ri][c0 + c] * R.DL[ri];
      for (int j = 0; j < kC; ++j) {
        const float kd = sKt[j][ri] * R.PE[j >> 4][ri];
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = fmaf(kd, sV[j][c0 + c], acc[c]);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) sS[ri][c0 + c] = acc[c];
    }
  }
  __syncthreads();
  if (ht) {
    for (int e = tid; e < 64 * kVT; e += kThreads) {
      const int kk = e / kVT, c = e % kVT;
      if (kk < K && v0 + c < V) ht[sb + static_cast<int64_t>(kk) * V + v0 + c] = sS[kk][c];
    }
  }
}

// --------------------------------------------------------------- backward --
// Workspace slot of the chunk starting at row t0 of sequence n:
// t0 / 64 + n is distinct for every chunk of every sequence when the
// sequences do not overlap (at most T / 64 + n_seq + 1 slots).
__device__ __forceinline__ int64_t state_slot(int64_t t0, int n) { return t0 / kC + n; }

__global__ __launch_bounds__(kThreads) void f32_bwd_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ g, const int64_t *__restrict__ cu, int n_seq, int64_t T, int H, int K, int V,
    float scale, const float *__restrict__ h0, const float *__restrict__ dO, const float *__restrict__ dht,
    float *__restrict__ dq, float *__restrict__ dk, float *__restrict__ dv, float *__restrict__ dg,
    float *__restrict__ dh0, float *__restrict__ hs, int64_t n_slots) {
  // sHQ holds the chunk's entering state h until its products are done,
  // then q~; sAD holds A until dv is done, then dA, then dG.
  __shared__ float sQ[kC][kP], sK[kC][kP], sKt[kC][kP], sHQ[kC][kP], sG[kC][kP];
  __shared__ float sV[kC][kP], sDO[kC][kP], sDH[64][kP], sAD[kC][kP];
  __shared__ ChunkRefs R;
  __shared__ float sDgH[64];   // 2^gamma sum_c dh h per key
  const int tid = threadIdx.x;
  const int h = static_cast<int>(blockIdx.x % H);
  const int n = static_cast<int>(blockIdx.x / H);
  int64_t bos, eos;
  seq_bounds(cu, n, T, bos, eos);
  const int64_t sb = (static_cast<int64_t>(n) * H + h) * K * V;
  const int ri = tid >> 2, q4 = tid & 3, c16 = 16 * q4;   // row (or key), and its 16 columns
  const int64_t nchunks = (eos - bos + kC - 1) / kC;
  auto slot_ptr = [&](int64_t t0) { return hs + (min(state_slot(t0, n), n_slots - 1) * H + h) * 64 * 64; };

  // ---- forward: the state entering every chunk -> workspace ----------------
  float S[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const int c = c16 + m;
    S[m] = (h0 && ri < K && c < V) ? h0[sb + static_cast<int64_t>(ri) * V + c] : 0.f;
  }
  for (int64_t ch = 0; ch < nchunks; ++ch) {
    const int64_t t0 = bos + ch * kC;
    const int nc = static_cast<int>(min(static_cast<int64_t>(kC), eos - t0));
    float *slot = slot_ptr(t0);
#pragma unroll
    for (int m = 0; m < 16; ++m) slot[ri * 64 + c16 + m] = S[m];
    __syncthreads();
    for (int e = tid; e < kC * 64; e += kThreads) {
      const int r = e >> 6, c = e & 63;
      const int64_t row = (t0 + r) * H + h;
      sK[r][c] = (r < nc && c < K) ? k[row * K + c] : 0.f;
      sG[r][c] = (r < nc && c < K) ? g[row * K + c] * kLog2e : 0.f;
      sV[r][c] = (r < nc && c < V) ? v[row * V + c] : 0.f;
    }
    __syncthreads();
    chunk_cumsum(sG, R);
    __syncthreads();
    chunk_tilde(nullptr, sK, sG, R, sKt, nullptr);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 16; ++m) S[m] *= R.DL[ri];
    for (int j = 0; j < kC; ++j) {
      const float kd = sKt[j][ri] * R.PE[j >> 4][ri];
#pragma unroll
      for (int m = 0; m < 16; ++m) S[m] = fmaf(kd, sV[j][c16 + m], S[m]);
    }
  }
  // ---- backward ----------------------------------------------------------------
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const int c = c16 + m;
    sDH[ri][c] = (dht && ri < K && c < V) ? dht[sb + static_cast<int64_t>(ri) * V + c] : 0.f;
  }
  for (int64_t ch = nchunks - 1; ch >= 0; --ch) {
    const int64_t t0 = bos + ch * kC;
    const int nc = static_cast<int>(min(static_cast<int64_t>(kC), eos - t0));
    const float *slot = slot_ptr(t0);
    __syncthreads();   // the previous (later) chunk is done with the tiles
    for (int e = tid; e < kC * 64; e += kThreads) {
      const int r = e >> 6, c = e & 63;
      const int64_t row = (t0 + r) * H + h;
      const bool okk = r < nc && c < K, okv = r < nc && c < V;
      sQ[r][c] = okk ? q[row * K + c] : 0.f;
      sK[r][c] = okk ? k[row * K + c] : 0.f;
      sG[r][c] = okk ? g[row * K + c] * kLog2e : 0.f;
      sV[r][c] = okv ? v[row * V + c] : 0.f;
      sDO[r][c] = okv ? dO[row * V + c] : 0.f;
      sHQ[r][c] = slot[e];   // the state entering this chunk (keys x values)
    }
    __syncthreads();
    chunk_cumsum(sG, R);
    __syncthreads();
    chunk_tilde(nullptr, sK, sG, R, sKt, nullptr);
    __syncthreads();
    float da[16];   // dA_i,16J.. of thread (row ri, block q4), kept until A is read
    {
      float a[16];
      a_row16(sQ, sK, sKt, sG, R, K, ri, q4, scale, a);
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) da[jj] = 0.f;
      if (q4 <= (ri >> 4)) {
        for (int c = 0; c < V; ++c) {
          const float d = sDO[ri][c];
#pragma unroll
          for (int jj = 0; jj < 16; ++jj) da[jj] = fmaf(d, sV[16 * q4 + jj][c], da[jj]);
        }
      }
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        sAD[ri][16 * q4 + jj] = a[jj];
        if (16 * q4 + jj > ri) da[jj] = 0.f;
      }
    }
    __syncthreads();
    {   // dv_j = sum_{i >= j} A_ij dO_i + k_d,j dh: thread (row ri, 16 columns)
      float acc[16];
#pragma unroll
      for (int m = 0; m < 16; ++m) acc[m] = 0.f;
      for (int i = ri; i < kC; ++i) {
        const float aij = sAD[i][ri];
#pragma unroll
        for (int m = 0; m < 16; ++m) acc[m] = fmaf(aij, sDO[i][c16 + m], acc[m]);
      }
      const int J = ri >> 4;
      for (int kk = 0; kk < K; ++kk) {
        const float kd = sKt[ri][kk] * R.PE[J][kk];
#pragma unroll
        for (int m = 0; m < 16; ++m) acc[m] = fmaf(kd, sDH[kk][c16 + m], acc[m]);
      }
      if (ri < nc) {
#pragma unroll
        for (int m = 0; m < 16; ++m)
          if (c16 + m < V) dv[((t0 + ri) * H + h) * V + c16 + m] = acc[m];
      }
    }
    __syncthreads();   // A is read: dA takes its place
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) sAD[ri][16 * q4 + jj] = da[jj];
    __syncthreads();
    // dq and dk of row ri, keys c16 .. c16 + 15 (the same thread holds both, so
    // dG = q dq - k dk needs no exchange)
    float qdq[16], kdk[16], tdk[16];
    {
      const int I = ri >> 4;
      float P[16], Ro[16];
#pragma unroll
      for (int m = 0; m < 16; ++m) P[m] = Ro[m] = 0.f;
      for (int c = 0; c < V; ++c) {   // P = dO_i . h_k
        const float d = sDO[ri][c];
#pragma unroll
        for (int m = 0; m < 16; ++m) P[m] = fmaf(d, sHQ[c16 + m][c], P[m]);
      }
      for (int J = 0; J < I; ++J) {   // blocks J < I: 2^(G_i - E_J) sum_j dA_ij k~_j
        float r[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) r[m] = 0.f;
        for (int j = 16 * J; j < 16 * J + 16; ++j) {
          const float d = sAD[ri][j];
#pragma unroll
          for (int m = 0; m < 16; ++m) r[m] = fmaf(d, sKt[j][c16 + m], r[m]);
        }
#pragma unroll
        for (int m = 0; m < 16; ++m) Ro[m] = fmaf(ex2c(sG[ri][c16 + m] - R.E[J][c16 + m]), r[m], Ro[m]);
      }
      for (int j = 16 * I; j < ri; ++j) {   // the diagonal block, term by term
        const float d = sAD[ri][j];
#pragma unroll
        for (int m = 0; m < 16; ++m)
          Ro[m] = fmaf(d * sK[j][c16 + m], ex2c(sG[ri][c16 + m] - sG[j][c16 + m]), Ro[m]);
      }
      // j = i adds s dA_ii k_i to dq and s dA_ii q_i to dk: equal terms of
      // q dq and k dk that cancel in dG, so dG is formed without them
      const float dii = sAD[ri][ri];
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const int kk = c16 + m;
        const float part = fmaf(ex2c(sG[ri][kk]), P[m], Ro[m]);
        qdq[m] = sQ[ri][kk] * (scale * part);
        const float dqv = scale * fmaf(dii, sK[ri][kk], part);
        if (ri < nc && kk < K) dq[((t0 + ri) * H + h) * K + kk] = dqv;
      }
    }
    if (tid < 64) {   // the state products are done with h: 2^gamma sum_c dh h
      float s = 0.f;
      for (int c = 0; c < V; ++c) s = fmaf(sDH[tid][c], sHQ[tid][c], s);
      sDgH[tid] = s * R.DL[tid];
    }
    __syncthreads();
    chunk_tilde(sQ, sK, sG, R, sKt, sHQ);   // q~ into sHQ (k~ again, unchanged)
    __syncthreads();
    {
      const int J = ri >> 4;
      float P[16], Ro[16];
#pragma unroll
      for (int m = 0; m < 16; ++m) P[m] = Ro[m] = 0.f;
      for (int c = 0; c < V; ++c) {   // P' = v_j . dh_k
        const float d = sV[ri][c];
#pragma unroll
        for (int m = 0; m < 16; ++m) P[m] = fmaf(d, sDH[c16 + m][c], P[m]);
      }
      for (int I = J + 1; I < 4; ++I) {   // blocks I > J: 2^(S_I - G_j) sum_i dA_ij q~_i
        float r[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) r[m] = 0.f;
        for (int i = 16 * I; i < 16 * I + 16; ++i) {
          const float d = sAD[i][ri];
#pragma unroll
          for (int m = 0; m < 16; ++m) r[m] = fmaf(d, sHQ[i][c16 + m], r[m]);
        }
#pragma unroll
        for (int m = 0; m < 16; ++m) Ro[m] = fmaf(ex2c(R.S[I][c16 + m] - sG[ri][c16 + m]), r[m], Ro[m]);
      }
      for (int i = ri + 1; i < 16 * J + 16; ++i) {   // the diagonal block, term by term
        const float d = sAD[i][ri];
#pragma unroll
        for (int m = 0; m < 16; ++m)
          Ro[m] = fmaf(d * sQ[i][c16 + m], ex2c(sG[i][c16 + m] - sG[ri][c16 + m]), Ro[m]);
      }
      const float dii = sAD[ri][ri];
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const int kk = c16 + m;
        const float kd = sKt[ri][kk] * R.PE[J][kk];                                      // k 2^(gamma - G)
        const float dkv = fmaf(ex2c(R.GAM[kk] - sG[ri][kk]), P[m], scale * fmaf(dii, sQ[ri][kk], Ro[m]));
        // the state term k 2^(gamma - G) P' enters dG here and dgamma with the
        // opposite sign: dG keeps the intra-chunk part, dg adds the state term
        // of the rows before t as a forward prefix
        kdk[m] = sK[ri][kk] * (scale * Ro[m]);
        tdk[m] = kd * P[m];
        if (ri < nc && kk < K) dk[((t0 + ri) * H + h) * K + kk] = dkv;
      }
    }
    __syncthreads();   // dA and k~ are no longer read
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      sAD[ri][c16 + m] = qdq[m] - kdk[m];   // dG
      sKt[ri][c16 + m] = tdk[m];
    }
    __syncthreads();
    if (tid < 64) {
      // dg_t = dgamma + sum_{r >= t} (q dq - k dk)_r with dgamma = 2^gamma
      // sum dh h + sum_j tdk_j; the tdk_r of rows r >= t cancel, so
      // dg_t = 2^gamma sum dh h + sum_{j < t} tdk_j + sum_{r >= t} dG_r
      const int kk = tid;
      float pre = 0.f;
      for (int j = 0; j < nc; ++j) {   // exclusive prefix of tdk, in place
        const float t = sKt[j][kk];
        sKt[j][kk] = pre;
        pre += t;
      }
      float acc = sDgH[kk];
      for (int r = nc - 1; r >= 0; --r) {
        acc += sAD[r][kk];
        if (kk < K) dg[((t0 + r) * H + h) * K + kk] = acc + sKt[r][kk];
      }
    }
    {   // dh <- 2^gamma dh + s sum_i (q 2^G)_i^T dO_i: thread (key ri, 16 columns);
        // only this thread reads or writes its dh entries from here on
      float acc[16];
#pragma unroll
      for (int m = 0; m < 16; ++m) acc[m] = sDH[ri][c16 + m] * R.DL[ri];
      for (int i = 0; i < kC; ++i) {
        const float qg = scale * sQ[i][ri] * ex2c(sG[i][ri]);
#pragma unroll
        for (int m = 0; m < 16; ++m) acc[m] = fmaf(qg, sDO[i][c16 + m], acc[m]);
      }
#pragma unroll
      for (int m = 0; m < 16; ++m) sDH[ri][c16 + m] = acc[m];
    }
  }
  __syncthreads();
  if (dh0) {
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const int c = c16 + m;
      if (ri < K && c < V) dh0[sb + static_cast<int64_t>(ri) * V + c] = sDH[ri][c];
    }
  }
}

inline int64_t f32_bwd_slots(int n_seq, int64_t T) { return T / kC + n_seq + 1; }

}  // namespace
}  // namespace ssla

extern "C" int ssla_gla_chunk_f32_fwd(const float *q, const float *k, const float *v, const float *g,
                                      const int64_t *cu_seqlens, int n_seq, int64_t T, int H, int K, int V,
                                      float scale, const float *h0, float *o, float *ht, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && T >= 0 && H > 0 && K > 0 && V > 0,
                 "gla_chunk_f32_fwd: bad sizes n_seq=%d T=%lld H=%d K=%d V=%d", n_seq, (long long)T, H, K, V);
  if (K > 64 || V > 256) {
    set_error("gla_chunk_f32_fwd: K=%d V=%d (K <= 64 and V <= 256 per call)", K, V);
    return SSLA_ERR_UNSUPPORTED;
  }
  if (n_seq == 0) return SSLA_OK;
  SSLA_CHECK_ARG(cu_seqlens && (T == 0 || (q && k && v && g && o)), "gla_chunk_f32_fwd: null pointer");
  const int nvt = (V + kVT - 1) / kVT;
  const int64_t blocks = static_cast<int64_t>(n_seq) * H * nvt;
  SSLA_CHECK_ARG(blocks < 0x7fffffff, "gla_chunk_f32_fwd: too many (sequence, head, tile) items");
  hipLaunchKernelGGL(f32_fwd_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), q, k, v, g, cu_seqlens, n_seq, T, H, K, V, scale, h0, o, ht);
  return launch_status("gla_chunk_f32_fwd");
}

extern "C" size_t ssla_gla_chunk_f32_bwd_workspace_size(int n_seq, int64_t T, int H) {
  if (n_seq < 0 || T < 0 || H <= 0) return 0;
  return static_cast<size_t>(ssla::f32_bwd_slots(n_seq, T)) * H * 64 * 64 * sizeof(float);
}

extern "C" int ssla_gla_chunk_f32_bwd(const float *q, const float *k, const float *v, const float *g,
                                      const int64_t *cu_seqlens, int n_seq, int64_t T, int H, int K, int V,
                                      float scale, const float *h0, const float *do_, const float *dht, float *dq,
                                      float *dk, float *dv, float *dg, float *dh0, void *workspace,
                                      size_t workspace_bytes, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && T >= 0 && H > 0 && K > 0 && V > 0,
                 "gla_chunk_f32_bwd: bad sizes n_seq=%d T=%lld H=%d K=%d V=%d", n_seq, (long long)T, H, K, V);
  if (K > 64 || V > 64) {
    set_error("gla_chunk_f32_bwd: K=%d V=%d (K, V <= 64 per call)", K, V);
    return SSLA_ERR_UNSUPPORTED;
  }
  if (n_seq == 0) return SSLA_OK;
  SSLA_CHECK_ARG(cu_seqlens && (T == 0 || (q && k && v && g && do_ && dq && dk && dv && dg)),
                 "gla_chunk_f32_bwd: null pointer");
  SSLA_CHECK_ARG(h0 == nullptr || dh0 != nullptr, "gla_chunk_f32_bwd: dh0 needed with an initial state");
  const size_t need = ssla_gla_chunk_f32_bwd_workspace_size(n_seq, T, H);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("gla_chunk_f32_bwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    return SSLA_ERR_WORKSPACE;
  }
  const int64_t blocks = static_cast<int64_t>(n_seq) * H;
  SSLA_CHECK_ARG(blocks < 0x7fffffff, "gla_chunk_f32_bwd: too many (sequence, head) items");
  hipLaunchKernelGGL(f32_bwd_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), q, k, v, g, cu_seqlens, n_seq, T, H, K, V, scale, h0, do_, dht,
                     dq, dk, dv, dg, dh0, static_cast<float *>(workspace), f32_bwd_slots(n_seq, T));
  return launch_status("gla_chunk_f32_bwd");
}
