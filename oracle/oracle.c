/*
 * oracle.c -- CPU restatement of the reference (haohq19/ssla) hot-path
 * arithmetic, used ONLY as the checker in tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg.  Nothing in the product (ssla_amd/)
 * links or calls it.
 *
 * All GLA / scan arithmetic is done in double precision on fp32 inputs, so
 * the oracle is more accurate than both the reference and the GPU path.
 * Build: python -m oracle.build  (gcc -O2 -shared -fPIC, -fopenmp).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define IDX3(t, h, d, H, D) (((int64_t)(t) * (H) + (h)) * (D) + (d))

/* naive_gla_recurrent (reference ops/gla/naive.py:50-111):
 *   S_t = exp(g_t)[:, None] * S_{t-1} + k_t v_t^T ;  o_t = (q_t * scale) . S_t
 * o_t uses the UPDATED state (naive.py:97-100).  h0 may be NULL (zeros,
 * naive.py:84-90); ht may be NULL (naive.py:103-104).  Parallel over
 * (sequence, head). */
void oracle_gla_recurrent(const float *q, const float *k, const float *v, const float *g,
                          const int64_t *cu, int n_seq, int H, int K, int V, double scale,
                          const float *h0, double *o, double *ht) {
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int n = 0; n < n_seq; ++n) {
    for (int h = 0; h < H; ++h) {
      double *S = (double *)malloc(sizeof(double) * K * V);
      for (int i = 0; i < K * V; ++i)
        S[i] = h0 ? (double)h0[((int64_t)n * H + h) * K * V + i] : 0.0;
      for (int64_t t = cu[n]; t < cu[n + 1]; ++t) {
        for (int kk = 0; kk < K; ++kk) {
          const double d = exp((double)g[IDX3(t, h, kk, H, K)]);
          const double kv = (double)k[IDX3(t, h, kk, H, K)];
          for (int vv = 0; vv < V; ++vv)
            S[kk * V + vv] = d * S[kk * V + vv] + kv * (double)v[IDX3(t, h, vv, H, V)];
        }
        for (int vv = 0; vv < V; ++vv) {
          double acc = 0.0;
          for (int kk = 0; kk < K; ++kk)
            acc += (double)q[IDX3(t, h, kk, H, K)] * scale * S[kk * V + vv];
          o[IDX3(t, h, vv, H, V)] = acc;
        }
      }
      if (ht)
        for (int i = 0; i < K * V; ++i) ht[((int64_t)n * H + h) * K * V + i] = S[i];
      free(S);
    }
  }
}

/* Backward of naive_gla_recurrent (the gradients that ChunkGLAFunction.
 * backward returns, reference ops/gla/chunk.py:1096-1116), fp64: with dS the
 * gradient of the state, walking t down from eos-1 (dS = dht, or 0):
 *   dS += scale q_t do_t^T;  dq_t = scale S_t do_t;  dk_t = dS v_t;
 *   dv_t = dS^T k_t;  dg_t[k] = e^{g_t[k]} sum_v dS[k,v] S_{t-1}[k,v];
 *   dS = diag(e^{g_t}) dS;   and dh0 = dS at the end.
 * States come from a forward pass with a checkpoint every 64 steps; each
 * block of 64 is recomputed forward before its reverse walk.  dh0 / dht may
 * be NULL.  Rows outside all sequences are left untouched. */
void oracle_gla_recurrent_bwd(const float *q, const float *k, const float *v, const float *g,
                              const int64_t *cu, int n_seq, int H, int K, int V, double scale,
                              const float *h0, const float *dout, const float *dht, double *dq,
                              double *dk, double *dv, double *dg, double *dh0) {
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int n = 0; n < n_seq; ++n) {
    for (int h = 0; h < H; ++h) {
      const int64_t bos = cu[n], eos = cu[n + 1], L = eos - bos;
      const int64_t nb = (L + 63) / 64;
      const size_t KV = (size_t)K * V;
      double *ck = (double *)malloc(sizeof(double) * KV * (size_t)(nb + 1));   /* state before each block */
      double *blk = (double *)malloc(sizeof(double) * KV * 65);                /* states of one block */
      double *dS = (double *)malloc(sizeof(double) * KV);
      double *S = (double *)malloc(sizeof(double) * KV);
      for (size_t i = 0; i < KV; ++i) S[i] = h0 ? (double)h0[((int64_t)n * H + h) * KV + i] : 0.0;
      for (int64_t b = 0; b < nb; ++b) {
        memcpy(ck + KV * b, S, sizeof(double) * KV);
        for (int64_t t = bos + 64 * b; t < bos + 64 * b + 64 && t < eos; ++t)
          for (int kk = 0; kk < K; ++kk) {
            const double d = exp((double)g[IDX3(t, h, kk, H, K)]), kv = (double)k[IDX3(t, h, kk, H, K)];
            for (int vv = 0; vv < V; ++vv)
              S[kk * V + vv] = d * S[kk * V + vv] + kv * (double)v[IDX3(t, h, vv, H, V)];
          }
      }
      for (size_t i = 0; i < KV; ++i) dS[i] = dht ? (double)dht[((int64_t)n * H + h) * KV + i] : 0.0;
      for (int64_t b = nb - 1; b >= 0; --b) {
        const int64_t t0 = bos + 64 * b, t1 = (t0 + 64 < eos) ? t0 + 64 : eos;
        memcpy(blk, ck + KV * b, sizeof(double) * KV);   /* blk[j] = state after row t0 + j - 1 */
        for (int64_t t = t0; t < t1; ++t) {
          double *P = blk + KV * (t - t0), *Q = P + KV;
          for (int kk = 0; kk < K; ++kk) {
            const double d = exp((double)g[IDX3(t, h, kk, H, K)]), kv = (double)k[IDX3(t, h, kk, H, K)];
            for (int vv = 0; vv < V; ++vv) Q[kk * V + vv] = d * P[kk * V + vv] + kv * (double)v[IDX3(t, h, vv, H, V)];
          }
        }
        for (int64_t t = t1 - 1; t >= t0; --t) {
          const double *St = blk + KV * (t - t0 + 1), *Sp = blk + KV * (t - t0);
          for (int kk = 0; kk < K; ++kk) {
            const double qs = (double)q[IDX3(t, h, kk, H, K)] * scale;
            for (int vv = 0; vv < V; ++vv) dS[kk * V + vv] += qs * (double)dout[IDX3(t, h, vv, H, V)];
          }
          for (int kk = 0; kk < K; ++kk) {
            double aq = 0.0, ak = 0.0, ag = 0.0;
            for (int vv = 0; vv < V; ++vv) {
              aq += St[kk * V + vv] * (double)dout[IDX3(t, h, vv, H, V)];
              ak += dS[kk * V + vv] * (double)v[IDX3(t, h, vv, H, V)];
              ag += dS[kk * V + vv] * Sp[kk * V + vv];
            }
            dq[IDX3(t, h, kk, H, K)] = scale * aq;
            dk[IDX3(t, h, kk, H, K)] = ak;
            dg[IDX3(t, h, kk, H, K)] = exp((double)g[IDX3(t, h, kk, H, K)]) * ag;
          }
          for (int vv = 0; vv < V; ++vv) {
            double a = 0.0;
            for (int kk = 0; kk < K; ++kk) a += dS[kk * V + vv] * (double)k[IDX3(t, h, kk, H, K)];
            dv[IDX3(t, h, vv, H, V)] = a;
          }
          for (int kk = 0; kk < K; ++kk) {
            const double d = exp((double)g[IDX3(t, h, kk, H, K)]);
            for (int vv = 0; vv < V; ++vv) dS[kk * V + vv] *= d;
          }
        }
      }
      if (dh0)
        for (size_t i = 0; i < KV; ++i) dh0[((int64_t)n * H + h) * KV + i] = dS[i];
      free(ck);
      free(blk);
      free(dS);
      free(S);
    }
  }
}

/* Chunked form of the same map, restating the reference forward pipeline
 * chunk_gla_fwd (reference ops/gla/chunk.py:906-960) with fp64 everywhere:
 *   1. G = chunk-local inclusive cumsum of g, restarting every BT rows of each
 *      sequence (ops/utils/cumsum.py:61-90, chunk indices ops/utils/index.py:69-77);
 *   2. entering state per chunk h[c]; S <- diag(e^{G_last}) S + (K e^{G_last-G})^T V
 *      (ops/common/chunk_h.py:66-123, chunk_h_naive.py:58-87);
 *   3. A_ij = scale sum_k q_ik k_jk e^{G_ik - G_jk}, j <= i (ops/gla/chunk.py:33-176);
 *   4. o = (q scale e^{G}) h[c] + tril(A) v (ops/gla/chunk.py:189-249).
 * Used to cross-check oracle_gla_recurrent (a different algorithm). */
void oracle_gla_chunk(const float *q, const float *k, const float *v, const float *g,
                      const int64_t *cu, int n_seq, int H, int K, int V, double scale,
                      const float *h0, int BT, double *o, double *ht) {
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int n = 0; n < n_seq; ++n) {
    for (int h = 0; h < H; ++h) {
      double *S = (double *)malloc(sizeof(double) * K * V);
      double *G = (double *)malloc(sizeof(double) * BT * K);
      double *A = (double *)malloc(sizeof(double) * BT * BT);
      for (int i = 0; i < K * V; ++i)
        S[i] = h0 ? (double)h0[((int64_t)n * H + h) * K * V + i] : 0.0;
      const int64_t bos = cu[n], eos = cu[n + 1];
      for (int64_t c0 = bos; c0 < eos; c0 += BT) {
        const int L = (int)((eos - c0) < BT ? (eos - c0) : BT);
        for (int kk = 0; kk < K; ++kk) {
          double run = 0.0;
          for (int i = 0; i < L; ++i) {
            run += (double)g[IDX3(c0 + i, h, kk, H, K)];
            G[i * K + kk] = run;
          }
        }
        for (int i = 0; i < L; ++i)
          for (int j = 0; j < L; ++j) {
            double a = 0.0;
            if (j <= i)
              for (int kk = 0; kk < K; ++kk)
                a += (double)q[IDX3(c0 + i, h, kk, H, K)] * (double)k[IDX3(c0 + j, h, kk, H, K)] *
                     exp(G[i * K + kk] - G[j * K + kk]);
            A[i * BT + j] = a * scale;
          }
        for (int i = 0; i < L; ++i)
          for (int vv = 0; vv < V; ++vv) {
            double acc = 0.0;
            for (int kk = 0; kk < K; ++kk)
              acc += (double)q[IDX3(c0 + i, h, kk, H, K)] * scale * exp(G[i * K + kk]) * S[kk * V + vv];
            for (int j = 0; j <= i; ++j) acc += A[i * BT + j] * (double)v[IDX3(c0 + j, h, vv, H, V)];
            o[IDX3(c0 + i, h, vv, H, V)] = acc;
          }
        const int last = L - 1;
        for (int kk = 0; kk < K; ++kk) {
          const double gl = G[last * K + kk];
          const double d = exp(gl);
          for (int vv = 0; vv < V; ++vv) {
            double acc = d * S[kk * V + vv];
            for (int j = 0; j < L; ++j)
              acc += (double)k[IDX3(c0 + j, h, kk, H, K)] * exp(gl - G[j * K + kk]) *
                     (double)v[IDX3(c0 + j, h, vv, H, V)];
            S[kk * V + vv] = acc;
          }
        }
      }
      if (ht)
        for (int i = 0; i < K * V; ++i) ht[((int64_t)n * H + h) * K * V + i] = S[i];
      free(S);
      free(G);
      free(A);
    }
  }
}

/* sequential_scan_fwd (reference ops/common/scan.py:20-43, :93-114):
 * h = zeros_like(u); per sequence and channel h_t = h_{t-1} * g_t + u_t with
 * h_{bos-1} = 0.  Rows outside all sequences stay 0. */
void oracle_diag_scan(const float *u, const float *g, const int64_t *cu, int n_seq, int64_t T,
                      int C, double *h) {
  memset(h, 0, sizeof(double) * (size_t)T * C);
#pragma omp parallel for schedule(dynamic)
  for (int n = 0; n < n_seq; ++n) {
    for (int c = 0; c < C; ++c) {
      double s = 0.0;
      for (int64_t t = cu[n]; t < cu[n + 1]; ++t) {
        s = s * (double)g[t * C + c] + (double)u[t * C + c];
        h[t * C + c] = s;
      }
    }
  }
}

/* sequential_scan_bwd (reference ops/common/scan.py:55-86): per sequence
 * and channel, t from eos-1 down to bos: dh += do_t; du_t = dh;
 * dg_t = dh * h_{t-1} (0 at bos); dh *= g_t.  h is the forward output
 * (recomputed here in fp64 from u, g).  Rows outside all sequences stay 0. */
void oracle_diag_scan_bwd(const float *u, const float *g, const float *dout, const int64_t *cu, int n_seq,
                          int64_t T, int C, double *du, double *dg) {
  memset(du, 0, sizeof(double) * (size_t)T * C);
  memset(dg, 0, sizeof(double) * (size_t)T * C);
#pragma omp parallel for schedule(dynamic)
  for (int n = 0; n < n_seq; ++n) {
    const int64_t bos = cu[n], eos = cu[n + 1];
    double *h = (double *)malloc(sizeof(double) * (size_t)(eos > bos ? eos - bos : 1));
    for (int c = 0; c < C; ++c) {
      double s = 0.0;
      for (int64_t t = bos; t < eos; ++t) {
        s = s * (double)g[t * C + c] + (double)u[t * C + c];
        h[t - bos] = s;
      }
      double dh = 0.0;
      for (int64_t t = eos - 1; t >= bos; --t) {
        dh += (double)dout[t * C + c];
        du[t * C + c] = dh;
        dg[t * C + c] = dh * (t > bos ? h[t - 1 - bos] : 0.0);
        dh *= (double)g[t * C + c];
      }
    }
    free(h);
  }
}

/* One bin of the per-site state update (naive_gla_recurrent on a length-1
 * sequence per active site, initial state = stored fp32 state, final state
 * stored back as fp32).  Inactive rows of `state` are not touched. */
void oracle_sparse_gla_step(const int32_t *site, int n_active, const float *q, const float *k,
                            const float *v, const float *g, float *state, int H, int K, int V,
                            double scale, double *o) {
#pragma omp parallel for collapse(2)
  for (int i = 0; i < n_active; ++i) {
    for (int h = 0; h < H; ++h) {
      float *S = state + ((int64_t)site[i] * H + h) * K * V;
      const int64_t io = (int64_t)i * H + h;
      double acc[256];
      for (int vv = 0; vv < V; ++vv) acc[vv] = 0.0;
      for (int kk = 0; kk < K; ++kk) {
        const double d = exp((double)g[io * K + kk]);
        const double kv = (double)k[io * K + kk];
        const double qs = (double)q[io * K + kk] * scale;
        for (int vv = 0; vv < V; ++vv) {
          const double s = d * (double)S[kk * V + vv] + kv * (double)v[io * V + vv];
          acc[vv] += qs * s;
          S[kk * V + vv] = (float)s;
        }
      }
      for (int vv = 0; vv < V; ++vv) o[io * V + vv] = acc[vv];
    }
  }
}

/* torch_scatter.scatter_max along dim 0 with a row index (documented
 * semantics; called at reference layers/sparse_pooling.py:33): events are
 * visited in index order, a strictly greater value replaces the running
 * maximum, so among equal maxima (floating-point ==) the smallest event
 * index wins; NaN never wins (a row whose values are all NaN counts as
 * empty).  Empty rows: out = 0, argmax = E.  out gets src[argmax]'s bits. */
void oracle_scatter_max(const float *src, const int64_t *index, int64_t E, int C, int64_t n_out,
                        float *out, int64_t *argmax) {
  for (int64_t i = 0; i < n_out * C; ++i) {
    out[i] = 0.f;
    argmax[i] = -1;
  }
  for (int64_t e = 0; e < E; ++e) {
    const int64_t r = index[e];
    for (int c = 0; c < C; ++c) {
      const float x = src[e * C + c];
      int64_t *a = &argmax[r * C + c];
      /* NaN never wins; ties keep the smallest e (events come in order) */
      if (x == x && (*a < 0 || x > src[*a * C + c])) *a = e;
    }
  }
  for (int64_t i = 0; i < n_out * C; ++i) {
    if (argmax[i] < 0) {
      argmax[i] = E;
      out[i] = 0.f;
    } else {
      out[i] = src[argmax[i] * C + (i % C)];
    }
  }
}

/* torch_scatter.scatter_mean along dim 0: sum / max(count, 1) (fp64 sum). */
void oracle_scatter_mean(const float *src, const int64_t *index, int64_t E, int C, int64_t n_out,
                         double *out) {
  int64_t *cnt = (int64_t *)calloc((size_t)(n_out > 0 ? n_out : 1), sizeof(int64_t));
  for (int64_t i = 0; i < n_out * C; ++i) out[i] = 0.0;
  for (int64_t e = 0; e < E; ++e) {
    const int64_t r = index[e];
    cnt[r] += 1;
    for (int c = 0; c < C; ++c) out[r * C + c] += (double)src[e * C + c];
  }
  for (int64_t r = 0; r < n_out; ++r) {
    const double d = (double)(cnt[r] > 0 ? cnt[r] : 1);
    for (int c = 0; c < C; ++c) out[r * C + c] /= d;
  }
  free(cnt);
}
