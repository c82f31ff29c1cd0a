// Varlen diagonal gated scan  h_t = g_t * h_{t-1} + u_t  (zero initial state).
//
// Semantics follow sequential_scan_fwd / SequentialScan.forward
// (reference ops/common/scan.py:20-43, :90-114): the state is fp32, restarts
// at every sequence start, and rows that belong to no sequence are zero.
//
// Layout: u, g, h (and do, du, dg of the backward) are fp32 [T, C].  A wavefront handles `slots` sequences at
// once when C is small (lanes = slot x channel), or one 64-channel slice of
// one sequence when C > 64.  Each step's loads do not depend on the state,
// so the loop prefetches kUnroll steps ahead; only the fma chain is serial.
#include "common.h"

namespace ssla {
namespace {

constexpr int kUnroll = 8;

__global__ __launch_bounds__(256) void diag_scan_kernel(
    const float *__restrict__ u, const float *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int64_t T, int C,
    int cw,            // channels per slot (power of two, <= 64)
    int n_cblk,        // channel blocks of width cw per sequence
    int64_t n_items,   // n_seq * n_cblk
    float *__restrict__ h) {
  const int lane = threadIdx.x & 63;
  const int slots = 64 / cw;
  const int slot = lane / cw;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t item = wave * slots + slot;
  if (item >= n_items) return;
  const int n = static_cast<int>(item / n_cblk);
  const int c = static_cast<int>(item % n_cblk) * cw + (lane % cw);
  if (c >= C) return;
  const int64_t bos = min(max(cu_seqlens[n], (int64_t)0), T);
  const int64_t eos = min(max(cu_seqlens[n + 1], bos), T);

  float state = 0.f;
  int64_t t = bos;
  for (; t + kUnroll <= eos; t += kUnroll) {
    float uu[kUnroll], gg[kUnroll];
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      uu[i] = u[(t + i) * C + c];
      gg[i] = g[(t + i) * C + c];
    }
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      state = fmaf(state, gg[i], uu[i]);
      h[(t + i) * C + c] = state;
    }
  }
  for (; t < eos; ++t) {
    state = fmaf(state, g[t * C + c], u[t * C + c]);
    h[t * C + c] = state;
  }
}

// Backward (sequential_scan_bwd, reference ops/common/scan.py:55-86): per
// sequence and channel, walking t down from eos - 1 to bos with dh = 0:
//   dh += do_t;  du_t = dh;  dg_t = dh * h_{t-1} (h_{bos-1} = 0);  dh *= g_t.
// The next step's "dh * g_t + do_{t-1}" is one fma.  Same wavefront layout
// and prefetch as the forward, in reverse.
__global__ __launch_bounds__(256) void diag_scan_bwd_kernel(
    const float *__restrict__ dout, const float *__restrict__ g, const float *__restrict__ h,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int64_t T, int C, int cw, int n_cblk,
    int64_t n_items, float *__restrict__ du, float *__restrict__ dg) {
  const int lane = threadIdx.x & 63;
  const int slots = 64 / cw;
  const int slot = lane / cw;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t item = wave * slots + slot;
  if (item >= n_items) return;
  const int n = static_cast<int>(item / n_cblk);
  const int c = static_cast<int>(item % n_cblk) * cw + (lane % cw);
  if (c >= C) return;
  const int64_t bos = min(max(cu_seqlens[n], (int64_t)0), T);
  const int64_t eos = min(max(cu_seqlens[n + 1], bos), T);

  float dh = 0.f, gn = 0.f;   // gn: g of the step after the current one
  int64_t t = eos;
  for (; t - kUnroll >= bos; t -= kUnroll) {
    float dd[kUnroll], gg[kUnroll], hp[kUnroll];
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      const int64_t s = t - 1 - i;
      dd[i] = dout[s * C + c];
      gg[i] = g[s * C + c];
      hp[i] = s > bos ? h[(s - 1) * C + c] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      const int64_t s = t - 1 - i;
      dh = fmaf(dh, gn, dd[i]);
      du[s * C + c] = dh;
      dg[s * C + c] = dh * hp[i];
      gn = gg[i];
    }
  }
  for (; t > bos; --t) {
    const int64_t s = t - 1;
    dh = fmaf(dh, gn, dout[s * C + c]);
    du[s * C + c] = dh;
    dg[s * C + c] = dh * (s > bos ? h[(s - 1) * C + c] : 0.f);
    gn = g[s * C + c];
  }
}

// Zero the rows before cu_seqlens[0] and from cu_seqlens[n_seq] on (all rows
// when n_seq == 0).  A kernel rather than hipMemsetAsync so that the call can
// be captured into a HIP graph.
__global__ __launch_bounds__(256) void diag_scan_zero_tail(
    const int64_t *__restrict__ cu_seqlens, int n_seq, int64_t T, int C,
    float *__restrict__ h) {
  const int64_t first = n_seq > 0 ? min(max(cu_seqlens[0], (int64_t)0), T) : T;
  const int64_t last = n_seq > 0 ? min(max(cu_seqlens[n_seq], first), T) : T;
  const int64_t head = first * C;
  const int64_t tail = (T - last) * C;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < head + tail;
       i += stride) {
    const int64_t idx = i < head ? i : last * C + (i - head);
    h[idx] = 0.f;
  }
}

}  // namespace
}  // namespace ssla

extern "C" int ssla_diag_scan_bwd(const float *dout, const float *g, const float *h, const int64_t *cu_seqlens,
                                  int n_seq, int64_t T, int C, float *du, float *dg, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && T >= 0 && C > 0, "diag_scan_bwd: bad sizes n_seq=%d T=%lld C=%d",
                 n_seq, (long long)T, C);
  if (T == 0) return SSLA_OK;
  SSLA_CHECK_ARG(dout && g && h && du && dg, "diag_scan_bwd: null tensor pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n_seq > 0) {
    SSLA_CHECK_ARG(cu_seqlens != nullptr, "diag_scan_bwd: cu_seqlens is NULL");
    int cw = 64;
    if (C <= 32) {
      cw = 1;
      while (cw < C) cw <<= 1;
    }
    const int n_cblk = (C + cw - 1) / cw;
    const int64_t n_items = static_cast<int64_t>(n_seq) * n_cblk;
    const int64_t blocks = ((n_items + 64 / cw - 1) / (64 / cw) + 3) / 4;
    if (blocks > 0x7fffffff) {
      set_error("diag_scan_bwd: too many sequences");
      return SSLA_ERR_UNSUPPORTED;
    }
    hipLaunchKernelGGL(diag_scan_bwd_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, dout, g, h,
                       cu_seqlens, n_seq, T, C, cw, n_cblk, n_items, du, dg);
  }
  // rows in no sequence: zero gradients (the reference's zeros_like)
  hipLaunchKernelGGL(diag_scan_zero_tail, dim3(64), dim3(256), 0, st, cu_seqlens, n_seq, T, C, du);
  hipLaunchKernelGGL(diag_scan_zero_tail, dim3(64), dim3(256), 0, st, cu_seqlens, n_seq, T, C, dg);
  return launch_status("diag_scan_bwd");
}

extern "C" int ssla_diag_scan_fwd(const float *u, const float *g, const int64_t *cu_seqlens,
                                  int n_seq, int64_t T, int C, float *h, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && T >= 0 && C > 0, "diag_scan_fwd: bad sizes n_seq=%d T=%lld C=%d",
                 n_seq, (long long)T, C);
  if (T == 0) return SSLA_OK;
  SSLA_CHECK_ARG(u && g && h, "diag_scan_fwd: null tensor pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n_seq == 0) {
    hipLaunchKernelGGL(diag_scan_zero_tail, dim3(64), dim3(256), 0, st, cu_seqlens, 0, T, C, h);
    return launch_status("diag_scan_fwd");
  }
  SSLA_CHECK_ARG(cu_seqlens != nullptr, "diag_scan_fwd: cu_seqlens is NULL");
  int cw = 64;
  if (C <= 32) {
    cw = 1;
    while (cw < C) cw <<= 1;
  }
  const int n_cblk = (C + cw - 1) / cw;
  const int64_t n_items = static_cast<int64_t>(n_seq) * n_cblk;
  const int slots = 64 / cw;
  const int64_t waves = (n_items + slots - 1) / slots;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks > 0x7fffffff) {
    set_error("diag_scan_fwd: too many sequences");
    return SSLA_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(diag_scan_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, u, g,
                     cu_seqlens, n_seq, T, C, cw, n_cblk, n_items, h);
  hipLaunchKernelGGL(diag_scan_zero_tail, dim3(64), dim3(256), 0, st, cu_seqlens, n_seq, T, C, h);
  return launch_status("diag_scan_fwd");
}
