/*
 * ssla_amd.h -- C-ABI of the MI355X (gfx950) SSLA hot-path library
 * (libssla_amd.so).
 *
 * Every entry point:
 *   - takes plain device pointers, element counts and a hipStream_t passed as
 *     `void *stream` (NULL = the default stream);
 *   - launches asynchronously on that stream and never synchronises the host;
 *   - never allocates or frees device memory: outputs and any workspace are
 *     owned by the caller, inputs are borrowed for the duration of the call;
 *   - returns an ssla_status (0 = OK, negative = error) and records a message
 *     retrievable with ssla_last_error() (thread-local).
 *
 * Layouts are packed "varlen" layouts: token-major [T_total, H, D] with
 * sequence boundaries given by an int64 cu_seqlens[N+1] array that lives on
 * the device (FlashAttention style).  All tensors must be contiguous.
 *
 * The reference this library replaces is Python + Triton (haohq19/ssla); each
 * declaration below cites the reference function it stands in for.
 */
#ifndef SSLA_AMD_H
#define SSLA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  SSLA_OK = 0,
  SSLA_ERR_ARG = -1,         /* bad shape, count or null pointer           */
  SSLA_ERR_DTYPE = -2,       /* dtype code not supported by this entry     */
  SSLA_ERR_WORKSPACE = -3,   /* workspace missing or smaller than required */
  SSLA_ERR_LAUNCH = -4,      /* hipGetLastError() reported a launch error  */
  SSLA_ERR_UNSUPPORTED = -5  /* shape outside what the kernels implement   */
} ssla_status;

typedef enum {
  SSLA_F32 = 0,
  SSLA_BF16 = 1,
  SSLA_F16 = 2
} ssla_dtype;

/* Library version (major*10000 + minor*100 + patch). */
int ssla_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char *ssla_last_error(void);

/* ------------------------------------------------------------------------
 * G1 -- gated linear attention (GLA) forward, varlen, vector (per-key) gates.
 *
 *   S_t = diag(exp(g_t)) S_{t-1} + k_t v_t^T        (per sequence, per head)
 *   o_t = (scale * q_t)^T S_t                       (o uses the UPDATED S_t)
 *
 * q, k: [T, H, K]; v, o: [T, H, V]  (all of dtype `dtype`)
 * g   : [T, H, K] log-gates, dtype `g_dtype` (F32 or the dtype of q)
 * cu_seqlens: int64 [n_seq + 1] on the device, non-decreasing,
 *             cu_seqlens[0] >= 0, cu_seqlens[n_seq] <= T.
 * h0  : fp32 [n_seq, H, K, V] initial states, or NULL for zeros.
 * ht  : fp32 [n_seq, H, K, V] final states, or NULL to skip.
 * Rows of o outside [cu_seqlens[0], cu_seqlens[n_seq]) are left untouched.
 * ------------------------------------------------------------------------ */

/* Chunked (chunk size 64) MFMA forward.  Replaces
 *   chunk_gla / ChunkGLAFunction.forward / chunk_gla_fwd
 *   (reference ops/gla/chunk.py:1119-1167, :1056-1094, :906-960)
 * together with chunk_local_cumsum (ops/utils/cumsum.py:346-364),
 * chunk_fwd_h (ops/common/chunk_h.py:242-294) and the intra-chunk /
 * output kernels (ops/gla/chunk.py:33-249, :644-743).  Supported: dtype
 * BF16 or F16, K == 64, V a multiple of 16 (<= 256).
 * Each sequence is split into segments processed in parallel; the
 * workspace (ssla_gla_chunk_workspace_size bytes, 16-byte aligned, no
 * initialisation needed) holds one fp32 state per segment.  A size of 0
 * means no workspace is needed for this shape (pass NULL, 0). */
size_t ssla_gla_chunk_workspace_size(int n_seq, int64_t T, int H, int K, int V);

int ssla_gla_chunk_fwd(const void *q, const void *k, const void *v,
                       const void *g, int g_dtype,
                       const int64_t *cu_seqlens, int n_seq, int64_t T,
                       int H, int K, int V, float scale,
                       const float *h0, void *o, float *ht, int dtype,
                       void *workspace, size_t workspace_bytes, void *stream);

/* Fused recurrent forward (state in registers, serial over t).  Same math
 * and signature as naive_gla_recurrent (reference ops/gla/naive.py:50-111).
 * Supported: dtype F32/BF16/F16, K <= 256, V <= 256.
 *
 * state_idx (int32 [n_seq] or NULL) optionally redirects sequence n's
 * initial and final state to row state_idx[n] of h0 / ht, which may then be
 * the SAME buffer (in-place per-site state update; rows not named by
 * state_idx are never read or written).  n_state_rows is the row count of
 * h0/ht when state_idx is given (a sequence whose state_idx is outside
 * [0, n_state_rows) is skipped).  This is the batched form of the per-site
 * sparse GLA step over many time bins.
 * Sequences are clamped to [0, T) on the device, so a malformed cu_seqlens
 * cannot address memory outside the tensors. */
int ssla_gla_recurrent_fwd(const void *q, const void *k, const void *v,
                           const void *g, int g_dtype,
                           const int64_t *cu_seqlens, int n_seq, int64_t T,
                           int H, int K, int V, float scale,
                           const float *h0, void *o, float *ht,
                           const int32_t *state_idx, int n_state_rows,
                           int dtype, void *stream);

/* ------------------------------------------------------------------------
 * G2 -- sparse sequential scans.
 * ------------------------------------------------------------------------ */

/* Varlen diagonal gated scan, zero initial state:
 *   h_t = g_t * h_{t-1} + u_t   per channel, restarting at every sequence.
 * u, g, h: fp32 [T, C].  Rows outside [cu_seqlens[0], cu_seqlens[n_seq])
 * are written with zeros (h is fully defined on return).  Replaces
 * scan / SequentialScan.forward / sequential_scan_fwd
 * (reference ops/common/scan.py:140-163, :90-114, :20-43). */
int ssla_diag_scan_fwd(const float *u, const float *g,
                       const int64_t *cu_seqlens, int n_seq, int64_t T,
                       int C, float *h, void *stream);

/* One time bin of the per-site matrix-state GLA update.  For active site
 * i (site = site_idx[i], sorted ascending, unique, < n_sites):
 *   S[site] <- diag(exp(g_i)) S[site] + k_i v_i^T ;  o_i = (scale q_i)^T S[site]
 * q, k, g: fp32 [n_active, H, K]; v, o: fp32 [n_active, H, V];
 * state: fp32 [n_sites, H, K, V], updated in place; rows of inactive sites
 * are neither read nor written.  No reference function exists for this
 * step; it is naive_gla_recurrent (ops/gla/naive.py:50-111) applied to a
 * length-1 sequence per active site with initial_state = S[site].
 * Supported: K, V in {16, 32, 64}. */
int ssla_sparse_gla_step(const int32_t *site_idx, int n_active,
                         const float *q, const float *k, const float *v,
                         const float *g, float *state, int n_sites, int H,
                         int K, int V, float scale, float *o, void *stream);

/* ------------------------------------------------------------------------
 * G3 -- scatter-reduce pooling (torch_scatter.scatter_max / scatter_mean
 * semantics along dim 0 with an index broadcast over channels, as called
 * at reference layers/sparse_pooling.py:33).
 *
 * src: fp32 [E, C]; index: int64 [E], every value in [0, n_out) (checked on
 * the device: an out-of-range index makes the call's status word report
 * SSLA_ERR_ARG via ssla_scatter_check, the offending row is skipped).
 *
 * scatter_max: out[n, c] = max over {e : index[e] = n} of src[e, c];
 *   argmax[n, c] = the SMALLEST such e attaining the maximum (floating-point
 *   comparison, so -0.0 == +0.0; out takes the bits of src[argmax]).
 *   Empty rows: out = 0, argmax = E.
 *   NaN values never win the comparison (a row whose values are all NaN
 *   reports out = 0, argmax = E).
 * scatter_mean: out[n, c] = sum / max(count, 1), summed in fp64 and
 *   rounded once; empty rows give 0.
 *
 * `index_sorted` = 1 promises index is non-decreasing (the segment ids that
 * unique_consecutive produces); the kernels then skip the bucketing pass.
 * Workspace: ssla_scatter_workspace_size(E, C, n_out) bytes (16-byte aligned,
 * no initialisation needed).  Any C >= 1; E below 2^31, n_out below 2^30.
 * Concurrent calls must use distinct workspaces.
 * ------------------------------------------------------------------------ */
size_t ssla_scatter_workspace_size(int64_t E, int C, int64_t n_out);

int ssla_scatter_max(const float *src, const int64_t *index, int64_t E,
                     int C, int64_t n_out, int index_sorted, float *out,
                     int64_t *argmax, void *workspace,
                     size_t workspace_bytes, void *stream);

int ssla_scatter_mean(const float *src, const int64_t *index, int64_t E,
                      int C, int64_t n_out, int index_sorted, float *out,
                      void *workspace, size_t workspace_bytes, void *stream);

/* Copies the device status word written by the last scatter call that used
 * `workspace` into *status_out (host), synchronising `stream`.  Returns
 * SSLA_OK; *status_out is SSLA_ERR_ARG if any index was out of range. */
int ssla_scatter_check(const void *workspace, int *status_out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SSLA_AMD_H */
