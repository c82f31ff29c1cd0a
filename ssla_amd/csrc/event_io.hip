// Event ingestion: Prophesee .dat Event2D records straight into the padded
// batch tensor the model consumes.
//
// Record (reference utils/io/dat_events_tools.py:15, :40-47): 8 bytes,
// uint32 t, then int32 w with x = w & 16383, y = (w & 268419072) >> 14,
// p = (w & 268435456) >> 28.  The batch (reference model_base.py:82-117,
// pad_batches): every sample's events as float32 rows, zero-padded to the
// longest sample; for Gen1 / NCaltech101 the columns are then reordered to
// <x, y, t, p> and p is mapped to 2p - 1 (padding rows included: they end
// as (0, 0, 0, -1)).  The float32 conversion of t
// rounds to nearest-even, as numpy's astype does.
//
// One thread per output row: one 8-byte record load, one 16-byte store (the
// padding rows store zeros).  HBM-bound: 8 B read + 16 B written per row.
#include "common.h"

namespace ssla {
namespace {

constexpr int kDecThreads = 256;

__global__ __launch_bounds__(kDecThreads) void dat_decode_kernel(const uint2 *__restrict__ rec,
                                                                 int64_t n_rec, const int64_t *__restrict__ start,
                                                                 int B, int64_t L, int layout,
                                                                 float4 *__restrict__ out) {
  const int64_t n_rows = static_cast<int64_t>(B) * L;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kDecThreads;
  const bool small = n_rows < 0x7fffffff;   // 32-bit division, not the 64-bit emulation
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * kDecThreads + threadIdx.x; g < n_rows; g += stride) {
    const int64_t b = small ? static_cast<int64_t>(static_cast<uint32_t>(g) / static_cast<uint32_t>(L)) : g / L;
    const int64_t i = g - b * L;
    const int64_t s0 = start[b], n = start[b + 1] - s0;
    // padding rows: zeros, then (Gen1 layout) p = 0 * 2 - 1 like every row
    float4 v = make_float4(0.f, 0.f, 0.f, layout == SSLA_EVENTS_XYTP ? -1.f : 0.f);
    if (i < n && s0 >= 0 && s0 + i < n_rec) {   // (rows outside the records: padding)
      const uint2 r = rec[s0 + i];
      const uint32_t w = r.y;
      const float t = static_cast<float>(r.x);   // round to nearest-even
      const float x = static_cast<float>(w & 16383u);
      const float y = static_cast<float>((w & 268419072u) >> 14);
      const float p = static_cast<float>((w & 268435456u) >> 28);
      v = layout == SSLA_EVENTS_XYTP ? make_float4(x, y, t, p * 2.f - 1.f) : make_float4(t, x, y, p);
    }
    out[g] = v;
  }
}

}  // namespace
}  // namespace ssla

extern "C" int ssla_dat_decode_batch(const void *records, int64_t n_records, const int64_t *sample_start, int B,
                                     int64_t max_len, int layout, float *events, void *stream) {
  ssla::clear_error();
  SSLA_CHECK_ARG(n_records >= 0 && B >= 0 && max_len >= 0, "dat_decode_batch: bad sizes n=%lld B=%d L=%lld",
                 (long long)n_records, B, (long long)max_len);
  SSLA_CHECK_ARG(layout == SSLA_EVENTS_XYTP || layout == SSLA_EVENTS_TXYP, "dat_decode_batch: bad layout %d",
                 layout);
  if (B == 0 || max_len == 0) return SSLA_OK;
  SSLA_CHECK_ARG(events && sample_start && (n_records == 0 || records), "dat_decode_batch: null pointer");
  SSLA_CHECK_ARG(ssla::aligned(records, 8) && ssla::aligned(events, 16) && ssla::aligned(sample_start, 8),
                 "dat_decode_batch: misaligned pointer");
  const int64_t n_rows = static_cast<int64_t>(B) * max_len;
  const int64_t blocks = std::min<int64_t>((n_rows + ssla::kDecThreads - 1) / ssla::kDecThreads, 65536);
  hipLaunchKernelGGL(ssla::dat_decode_kernel, dim3(static_cast<unsigned>(blocks)), dim3(ssla::kDecThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint2 *>(records), n_records,
                     sample_start, B, max_len, layout, reinterpret_cast<float4 *>(events));
  return ssla::launch_status("dat_decode_batch");
}
