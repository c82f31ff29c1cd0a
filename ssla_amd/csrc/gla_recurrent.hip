// Fused recurrent GLA forward (serial over time, state in registers).
//
// Semantics follow naive_gla_recurrent (reference ops/gla/naive.py:50-111):
//   S_t = exp(g_t)[:, None] * S_{t-1} + k_t v_t^T,   o_t = (scale q_t) . S_t
// with the initial state taken from h0 (or zero) and the final state written
// to ht.  One wavefront owns one (sequence, head, 16-column V tile); its 64
// lanes are 4 key-groups x 16 value columns, each lane holding KPL rows of
// the fp32 state.  The o reduction over the 4 key-groups is two xor-shuffles.
#include "common.h"

namespace ssla {
namespace {

constexpr int kBV = 16;   // value columns per wavefront
constexpr int kKG = 4;    // key groups per wavefront (64 / kBV)

// A sequence whose state row is outside [0, n_rows) or not above the row of
// the sequence before it (state_idx must be strictly increasing, so no two
// sequences share a state row) is skipped: its o rows are written as zeros,
// no state is read or written, and the status word is set to SSLA_ERR_ARG.
__device__ __forceinline__ bool bad_state_row(const int32_t *state_idx, int n, int64_t srow, int n_rows) {
  return state_idx && (srow < 0 || srow >= n_rows || (n > 0 && static_cast<int64_t>(state_idx[n - 1]) >= srow));
}

template <int DT>
__device__ __forceinline__ void skip_sequence(void *o, int64_t bos, int64_t eos, int H, int h, int V, int col,
                                              bool writer, int lane, int32_t *status) {
  if (writer)
    for (int64_t t = bos; t < eos; ++t) Elem<DT>::store(o, (t * H + h) * V + col, 0.f);
  if (status && lane == 0) __hip_atomic_store(status, SSLA_ERR_ARG, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// KPL consecutive elements of a row from index i into fp32: 16-byte loads
// for fp32, 8-byte loads for 16-bit types (i a multiple of KPL >= 4, base
// 16-byte aligned: checked by the host before this path is chosen).
template <int DT, int N>
__device__ __forceinline__ void load_run(const void *p, int64_t i, float (&x)[N]) {
  static_assert(N % 4 == 0, "runs of whole 4-element pieces");
  if constexpr (DT == SSLA_F32) {
    const float4 *s = reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
#pragma unroll
    for (int j = 0; j < N / 4; ++j) {
      const float4 t = s[j];
      x[4 * j] = t.x;
      x[4 * j + 1] = t.y;
      x[4 * j + 2] = t.z;
      x[4 * j + 3] = t.w;
    }
  } else {
    const uint2 *s = reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(p) + i);
#pragma unroll
    for (int j = 0; j < N / 4; ++j) {
      const uint2 u = s[j];
      const uint16_t e[4] = {static_cast<uint16_t>(u.x), static_cast<uint16_t>(u.x >> 16),
                             static_cast<uint16_t>(u.y), static_cast<uint16_t>(u.y >> 16)};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        x[4 * j + c] = DT == SSLA_BF16 ? bf16_bits_to_f32(e[c]) : f16_bits_to_f32(e[c]);
    }
  }
}

// Same recurrence for K == 4 * KPL with aligned rows: each lane's KPL keys
// are one contiguous run, loaded with vector loads, and the next step's
// q, k, g, v are in flight while the current step is computed.
template <int DT, int GDT, int KPL>
__global__ __launch_bounds__(256) void gla_recurrent_vec_kernel(
    const void *__restrict__ q, const void *__restrict__ k,
    const void *__restrict__ v, const void *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int H, int K, int V,
    float scale, const float *__restrict__ h0, void *__restrict__ o,
    float *__restrict__ ht, const int32_t *__restrict__ state_idx, int n_state_rows,
    int64_t T, int32_t *__restrict__ status) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int n_vt = (V + kBV - 1) / kBV;
  if (item >= static_cast<int64_t>(n_seq) * H * n_vt) return;  // whole wavefront exits
  const int vt = static_cast<int>(item % n_vt);
  const int h = static_cast<int>((item / n_vt) % H);
  const int n = static_cast<int>(item / (static_cast<int64_t>(n_vt) * H));
  const int col = vt * kBV + (lane & 15);
  const int k0 = (lane >> 4) * KPL;
  const bool col_ok = col < V;
  const int64_t bos = min(max(cu_seqlens[n], (int64_t)0), T);
  const int64_t eos = min(max(cu_seqlens[n + 1], bos), T);
  const int64_t srow = state_idx ? static_cast<int64_t>(state_idx[n]) : n;
  if (bad_state_row(state_idx, n, srow, n_state_rows)) {
    skip_sequence<DT>(o, bos, eos, H, h, V, col, (lane >> 4) == 0 && col_ok, lane, status);
    return;
  }

  float S[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) S[i] = (h0 && col_ok) ? h0[((srow * H + h) * K + k0 + i) * V + col] : 0.f;

  typedef Elem<DT> E;
  float qc[KPL], kc[KPL], gc[KPL], vc = 0.f;
  auto fetch = [&](int64_t t, float (&qx)[KPL], float (&kx)[KPL], float (&gx)[KPL], float &vx) {
    const int64_t base = (t * H + h) * K + k0;
    load_run<DT, KPL>(q, base, qx);
    load_run<DT, KPL>(k, base, kx);
    load_run<GDT, KPL>(g, base, gx);
    vx = col_ok ? E::load(v, (t * H + h) * V + col) : 0.f;
  };
  if (bos < eos) fetch(bos, qc, kc, gc, vc);
  for (int64_t t = bos; t < eos; ++t) {
    float qn[KPL], kn[KPL], gn[KPL], vn = 0.f;
    if (t + 1 < eos) fetch(t + 1, qn, kn, gn, vn);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      S[i] = fmaf(fast_exp2(gc[i] * kLog2e), S[i], kc[i] * vc);
      acc = fmaf(qc[i] * scale, S[i], acc);
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if ((lane >> 4) == 0 && col_ok) E::store(o, (t * H + h) * V + col, acc);
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      qc[i] = qn[i];
      kc[i] = kn[i];
      gc[i] = gn[i];
    }
    vc = vn;
  }
  if (ht && col_ok) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) ht[((srow * H + h) * K + k0 + i) * V + col] = S[i];
  }
}

template <int DT, int GDT, int KPL>
__global__ __launch_bounds__(256) void gla_recurrent_kernel(
    const void *__restrict__ q, const void *__restrict__ k,
    const void *__restrict__ v, const void *__restrict__ g,
    const int64_t *__restrict__ cu_seqlens, int n_seq, int H, int K, int V,
    float scale, const float *__restrict__ h0, void *__restrict__ o,
    float *__restrict__ ht, const int32_t *__restrict__ state_idx, int n_state_rows,
    int64_t T, int32_t *__restrict__ status) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int n_vt = (V + kBV - 1) / kBV;
  if (item >= static_cast<int64_t>(n_seq) * H * n_vt) return;  // whole wavefront exits
  const int vt = static_cast<int>(item % n_vt);
  const int h = static_cast<int>((item / n_vt) % H);
  const int n = static_cast<int>(item / (static_cast<int64_t>(n_vt) * H));

  const int col = vt * kBV + (lane & 15);   // value column of this lane
  const int kg = lane >> 4;                 // key group of this lane
  const int k0 = kg * KPL;                  // first key row of this lane
  const bool col_ok = col < V;

  // Clamp the sequence to [0, T) so that a malformed cu_seqlens can never
  // address memory outside q/k/v/g/o (the host wrapper reports it).
  const int64_t bos = min(max(cu_seqlens[n], (int64_t)0), T);
  const int64_t eos = min(max(cu_seqlens[n + 1], bos), T);
  const int64_t srow = state_idx ? static_cast<int64_t>(state_idx[n]) : n;
  if (bad_state_row(state_idx, n, srow, n_state_rows)) {   // never touch foreign rows
    skip_sequence<DT>(o, bos, eos, H, h, V, col, kg == 0 && col_ok, lane, status);
    return;
  }

  float S[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int kk = k0 + i;
    S[i] = (h0 && col_ok && kk < K) ? h0[((srow * H + h) * K + kk) * V + col] : 0.f;
  }

  typedef Elem<DT> E;
  typedef Elem<GDT> EG;
  for (int64_t t = bos; t < eos; ++t) {
    const int64_t qk_base = (t * H + h) * K;
    const float vv = col_ok ? E::load(v, (t * H + h) * V + col) : 0.f;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int kk = k0 + i;
      if (kk < K) {
        const float gg = EG::load(g, qk_base + kk);
        const float kv = E::load(k, qk_base + kk);
        const float qv = E::load(q, qk_base + kk);
        S[i] = fmaf(fast_exp2(gg * kLog2e), S[i], kv * vv);
        acc = fmaf(qv * scale, S[i], acc);
      }
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (kg == 0 && col_ok) E::store(o, (t * H + h) * V + col, acc);
  }

  if (ht && col_ok) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int kk = k0 + i;
      if (kk < K) ht[((srow * H + h) * K + kk) * V + col] = S[i];
    }
  }
}

template <int DT, int GDT>
int launch_recurrent(const void *q, const void *k, const void *v, const void *g,
                     const int64_t *cu, int n_seq, int H, int K, int V, float scale,
                     const float *h0, void *o, float *ht, const int32_t *sidx,
                     int n_rows, int64_t T, int32_t *status, hipStream_t st) {
  const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int n_vt = (V + kBV - 1) / kBV;
  const int64_t items = static_cast<int64_t>(n_seq) * H * n_vt;
  if (items == 0) return SSLA_OK;
  const int waves_per_block = 4;
  const int64_t blocks = (items + waves_per_block - 1) / waves_per_block;
  if (blocks > 0x7fffffff) {
    set_error("gla_recurrent_fwd: too many (sequence, head, tile) items");
    return SSLA_ERR_UNSUPPORTED;
  }
  dim3 grid(static_cast<unsigned>(blocks)), block(64 * waves_per_block);
  const int kpl_needed = (K + kKG - 1) / kKG;
  // vector path: every lane's run of keys is whole (K = 4 KPL), aligned, and
  // short enough to double-buffer in registers (K <= 64)
  const bool vec = (K % 16 == 0) && al16(q) && al16(k) && al16(g) && K <= 64;
  if (vec) {
#define SSLA_RECV(KPL_)                                                                        \
  hipLaunchKernelGGL((gla_recurrent_vec_kernel<DT, GDT, KPL_>), grid, block, 0, st, q, k, v, g, \
                     cu, n_seq, H, K, V, scale, h0, o, ht, sidx, n_rows, T, status)
    switch (K / kKG) {
      case 4: SSLA_RECV(4); return launch_status("gla_recurrent_fwd");
      case 8: SSLA_RECV(8); return launch_status("gla_recurrent_fwd");
      case 16: SSLA_RECV(16); return launch_status("gla_recurrent_fwd");
      default: break;   // other K: the general kernel
    }
#undef SSLA_RECV
  }
#define SSLA_REC(KPL_)                                                                     \
  hipLaunchKernelGGL((gla_recurrent_kernel<DT, GDT, KPL_>), grid, block, 0, st, q, k, v, g, \
                     cu, n_seq, H, K, V, scale, h0, o, ht, sidx, n_rows, T, status)
  if (kpl_needed <= 4) SSLA_REC(4);
  else if (kpl_needed <= 8) SSLA_REC(8);
  else if (kpl_needed <= 16) SSLA_REC(16);
  else if (kpl_needed <= 32) SSLA_REC(32);
  else SSLA_REC(64);
#undef SSLA_REC
  return launch_status("gla_recurrent_fwd");
}

}  // namespace
}  // namespace ssla

extern "C" int ssla_gla_recurrent_fwd(const void *q, const void *k, const void *v,
                                      const void *g, int g_dtype,
                                      const int64_t *cu_seqlens, int n_seq, int64_t T,
                                      int H, int K, int V, float scale,
                                      const float *h0, void *o, float *ht,
                                      const int32_t *state_idx, int n_state_rows,
                                      int32_t *status, int dtype, void *stream) {
  using namespace ssla;
  clear_error();
  SSLA_CHECK_ARG(n_seq >= 0 && T >= 0 && H > 0 && K > 0 && V > 0,
                 "gla_recurrent_fwd: bad sizes n_seq=%d T=%lld H=%d K=%d V=%d", n_seq,
                 (long long)T, H, K, V);
  if (K > 256 || V > 256) {
    set_error("gla_recurrent_fwd: K=%d V=%d exceed 256", K, V);
    return SSLA_ERR_UNSUPPORTED;
  }
  if (n_seq == 0) return SSLA_OK;
  SSLA_CHECK_ARG(cu_seqlens != nullptr, "gla_recurrent_fwd: cu_seqlens is NULL");
  SSLA_CHECK_ARG(T == 0 || (q && k && v && g && o), "gla_recurrent_fwd: null tensor pointer");
  SSLA_CHECK_ARG(state_idx == nullptr || n_state_rows > 0,
                 "gla_recurrent_fwd: state_idx given with n_state_rows=%d", n_state_rows);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SSLA_F32) {
    if (g_dtype != SSLA_F32) { set_error("gla_recurrent_fwd: fp32 inputs need fp32 g"); return SSLA_ERR_DTYPE; }
    return launch_recurrent<SSLA_F32, SSLA_F32>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, st);
  }
  if (dtype == SSLA_BF16) {
    if (g_dtype == SSLA_F32)
      return launch_recurrent<SSLA_BF16, SSLA_F32>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, st);
    if (g_dtype == SSLA_BF16)
      return launch_recurrent<SSLA_BF16, SSLA_BF16>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, st);
  }
  if (dtype == SSLA_F16) {
    if (g_dtype == SSLA_F32)
      return launch_recurrent<SSLA_F16, SSLA_F32>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, st);
    if (g_dtype == SSLA_F16)
      return launch_recurrent<SSLA_F16, SSLA_F16>(q, k, v, g, cu_seqlens, n_seq, H, K, V, scale, h0, o, ht, state_idx, n_state_rows, T, status, st);
  }
  set_error("gla_recurrent_fwd: unsupported dtype %d / g_dtype %d", dtype, g_dtype);
  return SSLA_ERR_DTYPE;
}
