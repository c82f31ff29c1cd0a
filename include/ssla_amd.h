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

/* Status words.  Entry points that validate data only the device sees
 * (index lists) take an optional `int32_t *status` in device memory: the
 * kernels store SSLA_ERR_ARG there when they find a bad entry and never
 * write it otherwise, so the caller sets it to SSLA_OK before the call.
 * ssla_status_read copies it to *value_out, synchronising `stream`. */
int ssla_status_read(const int32_t *status, int *value_out, void *stream);

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
 * BF16 or F16, K == 64, V a multiple of 16 (<= 256) -- other key widths
 * run as groups of 64 keys (the last one zero-padded) whose o add up, since
 * each key's decay only touches its own state row; one sequence below
 * 2^31 bytes per tensor (rows * H * max(K, V) * 4), SSLA_ERR_UNSUPPORTED
 * otherwise.  Only a batch with T * H * max(K, V) * 4 >= 2^31 can hold such
 * a sequence: then cu_seqlens is read back to check (one host
 * synchronisation).
 * Each sequence is split into segments processed in parallel; the
 * workspace (ssla_gla_chunk_workspace_size bytes, 16-byte aligned, no
 * initialisation needed) holds one bf16 hi / lo state pair (as the
 * reference stores its per-chunk states, ops/gla/chunk.py:933) and one
 * fp32 decay row per segment.  A size of 0
 * means no workspace is needed for this shape (pass NULL, 0). */
size_t ssla_gla_chunk_workspace_size(int n_seq, int64_t T, int H, int K, int V);

int ssla_gla_chunk_fwd(const void *q, const void *k, const void *v,
                       const void *g, int g_dtype,
                       const int64_t *cu_seqlens, int n_seq, int64_t T,
                       int H, int K, int V, float scale,
                       const float *h0, void *o, float *ht, int dtype,
                       void *workspace, size_t workspace_bytes, void *stream);

/* Allocation-free variant of ssla_gla_chunk_fwd (same arguments without
 * the workspace, same kernels, same results bit for bit).  It has no
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The workspace is a static device array
 * of 64 MiB inside the library, one copy per GPU, held until the process
 * ends; a shape whose ssla_gla_chunk_workspace_size exceeds it returns
 * SSLA_ERR_WORKSPACE.  Every call on one GPU uses that GPU's array, so calls
 * that overlap on one GPU (concurrent streams or host threads) race: run
 * them in one stream order.  The first call on a device looks the array's
 * address up (hipGetSymbolAddress); it allocates nothing. */
int ssla_gla_chunk_fwd_noalloc(const void *q, const void *k, const void *v,
                               const void *g, int g_dtype,
                               const int64_t *cu_seqlens, int n_seq, int64_t T,
                               int H, int K, int V, float scale,
                               const float *h0, void *o, float *ht, int dtype,
                               void *stream);

/* Chunked GLA in fp32: the forward and backward that chunk_gla runs for
 * fp32 inputs (reference chunk_gla_fwd / chunk_gla_bwd, ops/gla/chunk.py
 * 906-960 and 963-1053, which take any float dtype; the reference's dots
 * use TF32 operands, here every product is fp32).  q, k, g fp32 [T, H, K],
 * v fp32 [T, H, V], states fp32 [N, H, K, V] (h0 / ht / dht may be NULL),
 * o, dq, dk, dv, dg fp32 in the input layouts; rows outside
 * [cu_seqlens[0], cu_seqlens[n_seq]) are not written.  Chunks of 64 rows,
 * walked in order per (sequence, head): no serial walk over time steps.
 * Forward: K <= 64, V <= 256 per call (wider K: groups of 64 keys whose o
 * add up).  Backward: K, V <= 64 per call (wider K or V: groups of 64 keys
 * or value columns, as for the bf16 backward); dh0 is required with h0.
 * Workspace of the backward: ssla_gla_chunk_f32_bwd_workspace_size bytes
 * (every chunk's entering state; no initialisation needed); cu_seqlens
 * must be non-decreasing. */
int ssla_gla_chunk_f32_fwd(const float *q, const float *k, const float *v, const float *g,
                           const int64_t *cu_seqlens, int n_seq, int64_t T, int H, int K, int V,
                           float scale, const float *h0, float *o, float *ht, void *stream);
size_t ssla_gla_chunk_f32_bwd_workspace_size(int n_seq, int64_t T, int H);
int ssla_gla_chunk_f32_bwd(const float *q, const float *k, const float *v, const float *g,
                           const int64_t *cu_seqlens, int n_seq, int64_t T, int H, int K, int V,
                           float scale, const float *h0, const float *dout, const float *dht, float *dq,
                           float *dk, float *dv, float *dg, float *dh0, void *workspace,
                           size_t workspace_bytes, void *stream);

/* Backward of ssla_gla_chunk_fwd: ChunkGLAFunction.backward /
 * chunk_gla_bwd (reference ops/gla/chunk.py:1096-1116, 963-1053, with
 * chunk_bwd_dh, ops/common/chunk_h.py:145-239).  dout [T, H, V] (dtype of
 * v), dht [N, H, K, V] fp32 or NULL (no final-state gradient), h0 as in the
 * forward (NULL = zero).  Writes dq, dk [T, H, K] and dv [T, H, V] in the
 * input dtype, dg [T, H, K] in g's dtype, dh0 [N, H, K, V] fp32 (skipped when
 * NULL).  Rows outside [cu_seqlens[0], cu_seqlens[n_seq]) are not written.
 * Supported: dtype BF16 or F16, K == 64, V a multiple of 16 up to 64
 * (other key widths: per group of 64 keys, as in the forward, summing dv).
 * Workspace: ssla_gla_chunk_bwd_workspace_size bytes (16-byte aligned, no
 * initialisation needed): chunk offsets and two fp32 states per chunk
 * (every chunk's entering state and leaving-state gradient). */
size_t ssla_gla_chunk_bwd_workspace_size(int n_seq, int64_t T, int H, int K, int V);
int ssla_gla_chunk_bwd(const void *q, const void *k, const void *v,
                       const void *g, int g_dtype,
                       const int64_t *cu_seqlens, int n_seq, int64_t T,
                       int H, int K, int V, float scale, const float *h0,
                       const void *dout, const float *dht, void *dq, void *dk,
                       void *dv, void *dg, float *dh0, int dtype,
                       void *workspace, size_t workspace_bytes, void *stream);

/* Fused recurrent forward (state in registers, serial over t).  Same math
 * and signature as naive_gla_recurrent (reference ops/gla/naive.py:50-111).
 * Supported: dtype F32/BF16/F16, K <= 256, V <= 256.
 *
 * state_idx (int32 [n_seq] or NULL) optionally redirects sequence n's
 * initial and final state to row state_idx[n] of h0 / ht, which may then be
 * the SAME buffer (in-place per-site state update; rows not named by
 * state_idx are never read or written).  n_state_rows is the row count of
 * h0/ht when state_idx is given.  state_idx must be strictly increasing and
 * inside [0, n_state_rows) (so no two sequences share a state row): a
 * sequence whose entry is not is skipped -- its o rows are written as zeros,
 * no state is touched -- and SSLA_ERR_ARG is stored in *status (device
 * int32, may be NULL; see ssla_status_read).  This is the batched form of
 * the per-site sparse GLA step over many time bins.
 * Sequences are clamped to [0, T) on the device, so a malformed cu_seqlens
 * cannot address memory outside the tensors.  cu_seqlens must be
 * non-decreasing: with the segmented schedule below, sequences that overlap
 * can need more segments than the grid holds; the segments past it are not
 * run and SSLA_ERR_ARG is stored in *status.
 *
 * workspace (optional; NULL, 0 for none): with ssla_gla_recurrent_workspace_size
 * bytes (16-byte aligned, no initialisation needed) long sequences are cut
 * into 128-step segments that run in parallel -- a pass that leaves each
 * segment's local end state and decay, then one that folds them into every
 * segment's entering state (fp32 throughout) -- instead of one wavefront
 * walking the whole sequence.  The size query returns 0 for shapes where
 * the single pass is faster (sequences shorter than 64 steps on average)
 * or not available (K not a multiple of 16 up to 64); then pass NULL, 0. */
size_t ssla_gla_recurrent_workspace_size(int n_seq, int64_t T, int H, int K, int V);
int ssla_gla_recurrent_fwd(const void *q, const void *k, const void *v,
                           const void *g, int g_dtype,
                           const int64_t *cu_seqlens, int n_seq, int64_t T,
                           int H, int K, int V, float scale,
                           const float *h0, void *o, float *ht,
                           const int32_t *state_idx, int n_state_rows,
                           int32_t *status, int dtype, void *workspace,
                           size_t workspace_bytes, void *stream);

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

/* Its backward, given the forward's h and the output gradient dout:
 *   dh_t = dout_t + g_{t+1} dh_{t+1} (0 past the sequence end),
 *   du_t = dh_t,  dg_t = dh_t h_{t-1} (h_{bos-1} = 0);
 * du, dg: fp32 [T, C], rows outside every sequence written with zeros.
 * Replaces SequentialScan.backward / sequential_scan_bwd (reference
 * ops/common/scan.py:116-137, :55-86). */
int ssla_diag_scan_bwd(const float *dout, const float *g, const float *h,
                       const int64_t *cu_seqlens, int n_seq, int64_t T,
                       int C, float *du, float *dg, void *stream);

/* One time bin of the per-site matrix-state GLA update.  For active site
 * i (site = site_idx[i], strictly increasing, inside [0, n_sites)):
 *   S[site] <- diag(exp(g_i)) S[site] + k_i v_i^T ;  o_i = (scale q_i)^T S[site]
 * q, k, g: fp32 [n_active, H, K]; v, o: fp32 [n_active, H, V];
 * state: fp32 [n_sites, H, K, V], updated in place; rows of inactive sites
 * are neither read nor written.  No reference function exists for this
 * step; it is naive_gla_recurrent (ops/gla/naive.py:50-111) applied to a
 * length-1 sequence per active site with initial_state = S[site].
 * An entry that is out of range or not above the entry before it (a
 * duplicate, an unsorted list) is skipped: its o rows are written as zeros,
 * no state is touched, and SSLA_ERR_ARG is stored in *status (device int32,
 * may be NULL; see ssla_status_read).
 * Supported: K, V in {16, 32, 64}. */
int ssla_sparse_gla_step(const int32_t *site_idx, int n_active,
                         const float *q, const float *k, const float *v,
                         const float *g, float *state, int n_sites, int H,
                         int K, int V, float scale, float *o, int32_t *status,
                         void *stream);

/* Projections of the per-site GLA block of the asynchronous step (config
 * C5: ssla_amd.backbone.SiteGLABlock), each one launch on bf16 matrix
 * cores.  No reference function: the block is the C5 configuration's; the
 * rounding points are torch's bf16 F.linear (bf16 operands, fp32 sums, the
 * result rounded once to bf16).
 * ssla_site_project: x fp32 [n, cin]; w bf16 [4 hd, cin] (the rows of Wq,
 *   Wk, Wv, Wg in turn); q, k, v = bf16(bf16(x) W^T) as bf16 [n, hd];
 *   g = logsigmoid(bf16(bf16(x) Wg^T)) / gate_normalizer as fp32 [n, hd].
 *   cin a multiple of 32, hd a multiple of 32.
 * ssla_site_finish: o bf16 [n, hd]; wo bf16 [cout, hd]; x fp32 [n, cin];
 *   wr bf16 [cout, cin] or NULL (then cin == cout);
 *   y = LayerNorm(bf16(o Wo^T) + (bf16(bf16(x) Wr^T) or x)) * ln_w + ln_b
 *   (biased variance, eps inside the root), fp32 [n, cout].  hd, cin
 *   multiples of 32; cout in {16, 32, 64, 96, 128, 192, 256}.
 * x, o and the weights 16-byte aligned; SSLA_ERR_UNSUPPORTED for other
 * sizes. */
int ssla_site_project(const float *x, int64_t n, int cin, const uint16_t *w, int hd, float gate_normalizer,
                      uint16_t *q, uint16_t *k, uint16_t *v, float *g, void *stream);
int ssla_site_finish(const uint16_t *o, int64_t n, int hd, const uint16_t *wo, const float *x, int cin,
                     const uint16_t *wr, const float *ln_w, const float *ln_b, float eps, int cout, float *y,
                     void *stream);

/* The whole per-site GLA block (ssla_amd.backbone.SiteGLABlock.forward; no
 * reference function: the block is the C5 configuration's) on one window's
 * groups in one call: x fp32 [n, cin] (the groups' events, lengths[G] each,
 * in group order), the group coordinates gr_batch / gr_h / gr_w [G] of a
 * grid_h x grid_w grid, state fp32 [n_sites, heads, head_dim, head_dim]
 * updated in place at rows (b grid_h + h) grid_w + w, which must be strictly
 * increasing (else, as in ssla_gla_recurrent_fwd, the sequence is skipped
 * and SSLA_ERR_ARG stored in *status when status is not NULL).  Runs
 * ssla_site_project (w_qkvg bf16 [4 heads head_dim, cin]), the recurrence
 * of ssla_gla_recurrent_fwd with state_idx (bf16 q / k / v, fp32 gates,
 * bf16 o) and ssla_site_finish (w_o, w_r or NULL, ln_w, ln_b, eps) into
 * y fp32 [n, cout]; the sizes those calls support.  Workspace:
 * ssla_site_gla_block_workspace_size bytes (q, k, v, g, o, the offsets and
 * the recurrence's segment states). */
size_t ssla_site_gla_block_workspace_size(int64_t n, int64_t G, int heads, int head_dim);
int ssla_site_gla_block(const float *x, int64_t n, int cin, const int64_t *lengths, const int64_t *gr_batch,
                        const int64_t *gr_h, const int64_t *gr_w, int64_t G, int grid_h, int grid_w, float *state,
                        int n_sites, int heads, int head_dim, const uint16_t *w_qkvg, float gate_normalizer,
                        float scale, const uint16_t *w_o, const uint16_t *w_r, const float *ln_w, const float *ln_b,
                        float eps, int cout, float *y, int32_t *status, void *workspace, size_t workspace_bytes,
                        void *stream);

/* The detection head of the asynchronous step (ssla_amd.backbone.
 * DetectionHead, the YOLOX head's inference path: reference
 * layers/yolox_head.py:183-230 forward, :234-256 decode) over all levels in
 * one launch.  Per level: grid fp32 [batch, c, h, w] (rounded to bf16 as
 * the module's input); w_br bf16 [2 width, c] (the cls branch's 1x1
 * convolution rows, then the reg branch's); br_scale / br_shift fp32
 * [2 width] (eval-mode batch norm and the convolution bias folded: f =
 * SiLU(acc * scale + shift)); w_pred bf16 [16, 2 width] (rows: 4 box, 1
 * objectness, then the classes; zero where a prediction does not read a
 * branch) and b_pred fp32 [16]; stride.  out bf16 [batch, sum h w, n_out]:
 * ((p0 + x) s, (p1 + y) s, exp(p2) s, exp(p3) s, p4, p5 ...) per cell in
 * row-major cell order, levels in turn.  width a multiple of 16 up to 256,
 * c a multiple of 32, 5 <= n_out <= 16.  No reference C function. */
#define SSLA_HEAD_MAX_LEVELS 4
typedef struct {
  const float *grid;
  const uint16_t *w_br;
  const float *br_scale;
  const float *br_shift;
  const uint16_t *w_pred;
  const float *b_pred;
  int c, h, w, stride;
} ssla_head_level;
int ssla_detect_head(const ssla_head_level *levels, int n_levels, int batch, int n_out, int width, uint16_t *out,
                     void *stream);

/* ------------------------------------------------------------------------
 * G3 -- scatter-reduce pooling (torch_scatter.scatter_max / scatter_mean
 * semantics along dim 0 with an index broadcast over channels, as called
 * at reference layers/sparse_pooling.py:33).
 *
 * src: fp32 [E, C]; index: int64 [E], every value in [0, n_out) (checked on
 * the device: an out-of-range index makes the call's status word report
 * SSLA_ERR_ARG via ssla_scatter_check; the unsorted path skips the event).
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
 * A broken promise or an out-of-range value is reported through the status
 * word (SSLA_ERR_ARG), and the sorted path's output is then unspecified.
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


/* ------------------------------------------------------------------------
 * G4 -- event-stream glue (grouping, receptive fields / patches, ordered
 * index-add, truncation, temporal dropout, pooling keys, dense grids).
 *
 * Calls whose output size depends on the data write their counts into the
 * first int64 words of their workspace and their input-error flag as an
 * int32 at byte 256; ssla_events_counts() copies them to the host
 * (synchronising the stream), or a caller copies those 260 bytes itself
 * without waiting.  Outputs are capacity-sized.  All
 * orderings are stable (ties keep enumeration order).
 * ------------------------------------------------------------------------ */

/* Lookup table of 'same'-padded receptive fields: for every field (row-major
 * over the output grid) the pixel index y*W + x of each kernel coordinate
 * (row-major), -1 for padding; outcoord (may be NULL) the <x, y> output
 * coordinate of each field.  Replaces compute_rf2pixels
 * (utils/farsecnn_utils.py:95-128) and get_patch2pixel_lut
 * (utils/async_utils.py:96-122).  ssla_rf_lut_shape gives the field count. */
int ssla_rf_lut_shape(int H, int W, int kh, int kw, int sh, int sw, int64_t *n_rf);
int ssla_rf_lut(int H, int W, int kh, int kw, int sh, int sw, int64_t *lut, int64_t *outcoord, void *stream);

/* Copies counts[0..n_counts) of the last data-dependent call that used
 * `workspace` and its input-error flag (1 if an index was out of range). */
int ssla_events_counts(const void *workspace, int64_t *counts_out, int n_counts, int *bad_out, void *stream);
/* ssla_events_counts without waiting: the same 260 bytes (counts as int64
 * from byte 0, the bad-input flag as int32 at byte 256) copied into
 * host_head, pinned host memory of at least 260 bytes, in stream order;
 * they are there once the stream has passed the call (e.g. an event
 * recorded after it has completed).  No reference C function. */
int ssla_events_counts_async(const void *workspace, void *host_head, void *stream);

/* Group padded events [B, N, C] (x, y, t, features...) with lengths[B] by
 * pixel b*H*W + y*W + x (stable), keeping the latest max_per_px events of
 * every pixel.  Outputs: features [cap, C-3], time [cap] (int64 of t), per
 * group batch / h / w / length [cap] with cap = B*N.  counts: [0] groups,
 * [1] kept events, [2] valid events.  Replaces group_events
 * (utils/farsecnn_utils.py:130-174; utils/async_utils.py:10-84). */
size_t ssla_group_events_workspace_size(int B, int64_t N);
int ssla_group_events(const float *events, const int64_t *lengths, int B, int64_t N, int C, int H, int W,
                      int max_per_px, float *out_events, int64_t *out_time, int64_t *gr_batch,
                      int64_t *gr_h, int64_t *gr_w, int64_t *gr_len, void *workspace,
                      size_t workspace_bytes, void *stream);

/* MosModel.preprocess_inputs (model_mos.py:173-209) in one call on events
 * [B, N, C] (x, y, t, p, ...): group_events of <x, y, t, t, p, ...> (the
 * latest max_per_px events per pixel), the per-pixel delay in feature
 * column 0 (min((t - t_prev) / 1e5, 1) in fp32, 1 for a group's first
 * event), then truncate_packed_sequence to the first hot_pixel_thres events
 * of every group (hot_pixel_thres <= 0: none).  Outputs as
 * ssla_group_events with features [cap, C-2]; counts (ssla_events_counts)
 * [0] groups, [1] kept events, [2] valid events.  Workspace:
 * ssla_group_events_workspace_size. */
int ssla_preprocess_events(const float *events, const int64_t *lengths, int B, int64_t N, int C, int H, int W,
                           int max_per_px, int64_t hot_pixel_thres, float *out_events, int64_t *out_time,
                           int64_t *gr_batch, int64_t *gr_h, int64_t *gr_w, int64_t *gr_len, void *workspace,
                           size_t workspace_bytes, void *stream);

/* Scatter of pixel groups into receptive fields / patches, the shared core
 * of gather_receptive_fields (utils/farsecnn_utils.py:177-265) and
 * scatter_group_events_to_patch (utils/async_utils.py:125-240).  Fields are
 * (b, rf) for b < B; a field is active when one of its pixels holds a group.
 * Its events are the runs of its active pixels in kernel-coordinate order,
 * stably sorted by time.  plan: counts [0] active fields, [1] field events,
 * [2] max time, [3] pixel runs not sorted by time (0: the sort-free fill
 * below applies).  fill (with those counts): per field event its source pixel
 * event, time (may be NULL) and kernel position; per active field its flat
 * index b*n_rf + rf and event count.  E_cap bounds the field events. */
size_t ssla_rf_scatter_workspace_size(int64_t G, int B, int H, int W, int64_t n_rf, int64_t E_cap);
int ssla_rf_scatter_plan(const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w,
                         const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in, int B,
                         int H, int W, const int64_t *lut, int64_t n_rf, int A, int64_t E_cap,
                         void *workspace, size_t workspace_bytes, void *stream);
int ssla_rf_scatter_fill(const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in, int B,
                         int H, int W, const int64_t *lut, int64_t n_rf, int A, int64_t E_cap,
                         int64_t n_active, int64_t E_out, int64_t t_max, int64_t *out_src,
                         int64_t *out_time, int64_t *out_pos, int64_t *f_index, int64_t *f_len,
                         void *workspace, size_t workspace_bytes, void *stream);

/* Sort-free fill for plans whose counts[3] is 0 (every pixel run
 * non-decreasing in time, as group_events and the field outputs leave them,
 * and E_in <= E_cap): the same outputs as ssla_rf_scatter_fill, each row
 * placed by counting the earlier events of the field's other runs.  inv
 * (H * W * A int32) is caller scratch; dst_map (E_in * A int32, may be NULL)
 * receives the row of every (event, kernel position) pair or -1. */
int ssla_rf_scatter_fill_sorted(const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w,
                                const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in, int B, int H,
                                int W, const int64_t *lut, int64_t n_rf, int A, int64_t E_cap, int64_t n_active,
                                int64_t E_out, int64_t *out_src, int64_t *out_time, int64_t *out_pos,
                                int64_t *f_index, int64_t *f_len, int32_t *inv, int32_t *dst_map, void *workspace,
                                size_t workspace_bytes, void *stream);

/* out[j, :] = src[idx[j], :] for rows of C floats (0 for idx out of range). */
int ssla_gather_rows(const float *src, int64_t n_src, const int64_t *idx, int64_t m, int C, float *out,
                     void *stream);

/* out[r, :] = sum of src rows i with idx[i] == r, added in increasing i from
 * zero in fp32: the arithmetic of index_add_ into zeros on the CPU.
 * Replaces gather_patch_events_to_group (utils/async_utils.py:243-264). */
size_t ssla_index_add_rows_workspace_size(int64_t n);
int ssla_index_add_rows(const float *src, const int64_t *idx, int64_t n, int C, int64_t n_out, float *out,
                        void *workspace, size_t workspace_bytes, void *stream);

/* Fused MosAttention forward (inference): everything of MosAttention.forward
 * (layers/mos_attention.py:75-140) after scatter_group_events_to_patch --
 * _apply_scatter_proj and _apply_gather_proj (:148-167), q/v/g projections,
 * sigmoid, scan (ops/common/scan.py:20-43), o_proj,
 * gather_patch_events_to_group (utils/async_utils.py:243-264), input_proj,
 * the residual and LayerNorm -- in three kernels with no intermediate sort.
 * Rows come from ssla_rf_scatter_fill (row_src, row_pos, patch_len of the
 * n_patches active patches; rows of a patch consecutive and in time order).
 * Weights fp32 as the reference module holds them: w_scatter
 * [A or 1, hidden, c_in] (scatter_per_pos = 0: one matrix), w_q/w_v/w_g/w_o
 * [hidden, hidden], w_gather [A or 1, hidden, hidden], w_in [hidden, c_in]
 * or NULL (then c_in == hidden), ln_w/ln_b [hidden], eps.  out [n_events,
 * hidden].  Supports c_in, hidden <= 32, A <= 49 and weights that fit 64 KB
 * of LDS (ssla_mos_attention_lds_bytes); SSLA_ERR_UNSUPPORTED otherwise. */
size_t ssla_mos_attention_workspace_size(int64_t n_events, int c_in, int hidden, int A, int64_t n_rows,
                                         int64_t n_patches);
size_t ssla_mos_attention_lds_bytes(int c_in, int hidden, int A, int scatter_per_pos, int gather_per_pos);
int ssla_mos_attention_fwd(const float *events, int64_t n_events, int c_in, const int64_t *row_src,
                           const int64_t *row_pos, int64_t n_rows, const int64_t *patch_len, int64_t n_patches,
                           int A, const float *w_scatter, int scatter_per_pos, const float *w_q, const float *w_v,
                           const float *w_g, const float *w_o, const float *w_gather, int gather_per_pos,
                           const float *w_in, const float *ln_w, const float *ln_b, float eps, int hidden,
                           float *out, void *workspace, size_t workspace_bytes, void *stream);

/* Stable sort of (uint64 key, int32 value) pairs on the low end_bit key
 * bits; vals_in NULL means 0..n-1.  Used for the (batch, time) ordering of
 * LinearAttention.forward (layers/linear_attention.py:62-63) and the
 * position bucketing of the patch projections (layers/mos_attention.py:148-167). */
size_t ssla_sort_pairs_workspace_size(int64_t n);
int ssla_sort_pairs(const uint64_t *keys_in, const int32_t *vals_in, int64_t n, int end_bit,
                    uint64_t *keys_out, int32_t *vals_out, void *workspace, size_t workspace_bytes,
                    void *stream);

/* Workspace of the segment calls below (n_seq = number of segments; for
 * ssla_pool_segments max(n_f, E)). */
size_t ssla_segments_workspace_size(int64_t n_seq);

/* truncate_packed_sequence (utils/farsecnn_utils.py:8-33): keep the first
 * `threshold` rows of every sequence of data [E, C] (and of others [E]).
 * counts[0] = rows kept. */
int ssla_truncate_packed(const float *data, const int64_t *seqlens, int64_t n_seq, int64_t E, int C,
                         int64_t threshold, const int64_t *others, float *out_data, int64_t *out_lengths,
                         int64_t *out_others, void *workspace, size_t workspace_bytes, void *stream);

/* TemporalDropout.forward keep indices (layers/temporal_dropout.py:30-53):
 * ceil(len / window) rows per sequence, every window-th, the last kept.
 * counts[0] = rows kept; out_idx holds idx_cap rows (sum(len) + n_seq
 * always suffices) and a count above idx_cap means the rows past it were
 * not written: the caller reports that as an error. */
int ssla_temporal_dropout_index(const int64_t *lengths, int64_t n_seq, int64_t window, int64_t *out_idx,
                                int64_t idx_cap, int64_t *out_lengths, void *workspace, size_t workspace_bytes,
                                void *stream);

/* repeat_interleave(values, lengths) into out [n] (layers/linear_attention.py:60,
 * layers/sparse_pooling.py:27). */
int ssla_expand_segments(const int64_t *values, const int64_t *lengths, int64_t n_seq, int64_t n,
                         int64_t *out, void *workspace, size_t workspace_bytes, void *stream);

/* SparsePool keys (layers/sparse_pooling.py:26-48): events of a field with
 * equal time form one pooling segment.  seg[E] (non-decreasing: the sorted
 * index of ssla_scatter_max / _mean), seg_time / seg_field per segment,
 * new_lengths[n_f] segments per field, field[E] scratch.  counts[0] =
 * segments. */
int ssla_pool_segments(const int64_t *time, const int64_t *lengths, int64_t n_f, int64_t E, int64_t *field,
                       int64_t *seg, int64_t *seg_time, int64_t *seg_field, int64_t *new_lengths,
                       void *workspace, size_t workspace_bytes, void *stream);

/* SparsePool.forward (layers/sparse_pooling.py:14-48) on pixel groups with
 * its receptive-field gather (AsyncSparseModule.gather_receptive_fields,
 * layers/async_sparse_module.py:23-41 -> utils/farsecnn_utils.py:177-265)
 * in two calls, for callers that need no gradient: the field rows are never
 * stored as features, the reduction reads the pixel events [E_in, C]
 * through each row's source event.  E_cap bounds the field rows: E_in times
 * the fields one pixel can belong to (ceil(kh/sh) * ceil(kw/sw)); more rows
 * than that is SSLA_ERR_ARG, and E_cap == E_in (one field per pixel) takes
 * a fill with one thread per event (a pixel found in two fields is
 * SSLA_ERR_ARG).  plan: counts_out[0] active fields, [1]
 * pooling segments, [2] field rows, [3] 1 if a group coordinate or run is
 * out of range (nothing else computed); it reads counts from the device
 * once (twice when a pixel run is not sorted by time).  emit (same
 * workspace and sizes, mode 0 scatter_max / 1 scatter_mean): out_events
 * [segments, C], out_time [segments], and per active field out_len
 * (segments), out_batch, out_h, out_w (outcoord [n_rf, 2] holds (w, h) per
 * field) -- the dict SparsePool.forward returns.  The values (out_events)
 * and the structure (out_time and the per-field outputs) may be emitted by
 * two calls on the same plan: a null out_events skips the values, a null
 * out_len skips the structure (both null: nothing is written), so the
 * structure of a window can be planned before its values exist. */
size_t ssla_sparse_pool_workspace_size(int64_t G, int64_t E_in, int B, int H, int W, int64_t n_rf, int A,
                                       int64_t E_cap);
int ssla_sparse_pool_plan(const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w,
                          const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in, int B, int H,
                          int W, const int64_t *lut, int64_t n_rf, int A, int64_t E_cap, int64_t *counts_out,
                          void *workspace, size_t workspace_bytes, void *stream);
/* The plan in two halves, for callers that keep the device busy while the
 * counts travel back: plan_enqueue launches the plan's kernels and reads
 * nothing (the counts land in the first bytes of the workspace, where
 * ssla_events_counts reads them; the caller may copy those bytes to host
 * memory asynchronously on the same stream); plan_finish takes head[0..5]
 * and bad as ssla_events_counts returns them once the enqueue's kernels are
 * done, checks them and, when a pixel run is not sorted by time, runs the
 * sort fill (two more reads).  counts_out as for plan.  The same
 * reference interface as plan (layers/sparse_pooling.py:14-48). */
int ssla_sparse_pool_plan_enqueue(const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w,
                                  const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in, int B,
                                  int H, int W, const int64_t *lut, int64_t n_rf, int A, int64_t E_cap,
                                  void *workspace, size_t workspace_bytes, void *stream);
int ssla_sparse_pool_plan_finish(const int64_t *gr_len, int64_t G, const int64_t *time, int64_t E_in, int B,
                                 int H, int W, const int64_t *lut, int64_t n_rf, int A, int64_t E_cap,
                                 const int64_t *head, int bad, int64_t *counts_out, void *workspace,
                                 size_t workspace_bytes, void *stream);
int ssla_sparse_pool_emit(const float *events, int C, int64_t G, int64_t E_in, int B, int H, int W, int64_t n_rf,
                          int A, int64_t E_cap, const int64_t *outcoord, int mode, int64_t n_act, int64_t n_seg,
                          int64_t E_out, float *out_events, int64_t *out_time, int64_t *out_len,
                          int64_t *out_batch, int64_t *out_h, int64_t *out_w, void *workspace,
                          size_t workspace_bytes, void *stream);

/* The values half of ssla_sparse_pool_emit for events that are a bf16
 * linear map of K = 2 inputs (a stem embedding nn.Linear(2, C, bias=False)
 * run as F.linear(x.bfloat16(), w.bfloat16()).float() before the pooling):
 * x fp32 [E_in, 2] (8-byte aligned), w bf16 [C, 2], C a multiple of 4.
 * out_events [n_seg, C] equals ssla_sparse_pool_emit on the mapped events
 * bit for bit: inputs and results rounded to bf16 (nearest-even), the two
 * products exact in fp32 and their sum rounded once.  No reference C
 * function (the reference runs the embedding and the pooling apart). */
int ssla_sparse_pool_emit_linear(const float *x, int K, const uint16_t *w, int C, int64_t G, int64_t E_in, int B,
                                 int H, int W, int64_t n_rf, int A, int64_t E_cap, int mode, int64_t n_act,
                                 int64_t n_seg, int64_t E_out, float *out_events, void *workspace,
                                 size_t workspace_bytes, void *stream);

/* Per-pixel delays in place (MosModel.preprocess_inputs, model_mos.py:
 * 195-201): column 0 of feat [E, C] (timestamps) becomes
 * min((t_i - t_(i-1)) / 1e5, 1) within each group, 1 at each group start. */
int ssla_pixel_delays(float *feat, int64_t E, int C, const int64_t *lengths, int64_t G, void *workspace,
                      size_t workspace_bytes, void *stream);

/* async_event_to_grid (model_mos.py:212-228): the last event of every group
 * at its (b, h, w) cell of grid [B, C, Hg, Wg]; other cells untouched. */
int ssla_events_to_grid(const float *events, int64_t E, int C, const int64_t *lengths,
                        const int64_t *gr_batch, const int64_t *gr_h, const int64_t *gr_w, int64_t G, int B,
                        int Hg, int Wg, float *grid, void *workspace, size_t workspace_bytes, void *stream);

/* async_event_to_grid (model_mos.py:212-228) for several levels in one
 * launch, each grid [B, C, Hg, Wg] written whole: the last event of every
 * group at its cell, 0 elsewhere (the reference's index_add_ into zeros,
 * one group per cell).  No workspace.  status (optional, device int32) is
 * set to 1 when a group's cell or last event lies out of range (that group
 * is skipped).  Each level needs B * Hg * Wg <= SSLA_GRIDS_MAX_CELLS. */
#define SSLA_GRIDS_MAX_LEVELS 8
#define SSLA_GRIDS_MAX_CELLS 16384
typedef struct {
  const float *events;
  const int64_t *lengths;
  const int64_t *batch;
  const int64_t *h;
  const int64_t *w;
  float *grid;
  int64_t E, G;
  int C, Hg, Wg;
} ssla_grid_level;
int ssla_events_to_grids(const ssla_grid_level *levels, int n_levels, int B, int32_t *status, void *stream);

/* ------------------------------------------------------------------------
 * Event ingestion: Prophesee .dat Event2D records -> the padded batch
 * tensor (reference utils/io/dat_events_tools.py:15,40-47 record decode;
 * model_base.py:82-117 pad_batches).
 *
 * records: device copy of n_records raw 8-byte records (uint32 t, int32 w:
 * x = w & 16383, y = (w >> 14) & 16383, p = (w >> 28) & 1), 8-byte aligned.
 * sample_start: device int64 [B + 1], non-decreasing, sample b's records are
 * [sample_start[b], sample_start[b+1]) (rows outside [0, n_records) are
 * treated as padding).  events: device float32 [B, max_len, 4], 16-byte
 * aligned.  layout SSLA_EVENTS_XYTP (Gen1 / NCaltech101): rows (x, y, t,
 * 2p - 1), padding rows (0, 0, 0, -1); SSLA_EVENTS_TXYP: rows (t, x, y, p),
 * padding rows 0.  t is converted to float32 with round-to-nearest-even.
 * ------------------------------------------------------------------------ */
enum { SSLA_EVENTS_XYTP = 0, SSLA_EVENTS_TXYP = 1 };
int ssla_dat_decode_batch(const void *records, int64_t n_records, const int64_t *sample_start, int B,
                          int64_t max_len, int layout, float *events, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SSLA_AMD_H */
