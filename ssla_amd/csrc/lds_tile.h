// Swizzled 64 x 64 tiles of 16-bit values in LDS and the MFMA operand reads
// of them (shared by the chunked GLA forward and backward kernels).
#pragma once
#include "common.h"

namespace ssla {

typedef short s16x4 __attribute__((ext_vector_type(4)));

template <class V8>
__device__ __forceinline__ V8 from_bits(const uint4 &x) { return __builtin_bit_cast(V8, x); }
template <class V8>
__device__ __forceinline__ uint4 to_bits(const V8 &x) { return __builtin_bit_cast(uint4, x); }

// A tile is [64 rows][64 columns] of 16-bit values, rows of 128 bytes, with
// the 16-byte segments of row r permuted by XOR (r & 7) so that the column
// reads of the MFMA operand layouts spread over the banks.
__device__ __forceinline__ int swz(int row, int col) {
  return row * 64 + ((((col >> 3) ^ (row & 7)) << 3) | (col & 7));
}

// 16 bytes (8 consecutive columns from col, col % 8 == 0) of one row.
__device__ __forceinline__ uint4 tile_row8(const uint16_t *t, int row, int col) {
  return *reinterpret_cast<const uint4 *>(t + swz(row, col));
}
__device__ __forceinline__ void tile_store8(uint16_t *t, int row, int col, const uint4 &x) {
  *reinterpret_cast<uint4 *>(t + swz(row, col)) = x;
}
// 8 bytes (4 consecutive columns from col, col % 4 == 0) of one row.
__device__ __forceinline__ uint2 tile_row4(const uint16_t *t, int row, int col) {
  return *reinterpret_cast<const uint2 *>(t + swz(row, col));
}
__device__ __forceinline__ void tile_store4(uint16_t *t, int row, int col, const uint2 &x) {
  *reinterpret_cast<uint2 *>(t + swz(row, col)) = x;
}

// ds_read_b64_tr_b16 lane mapping (16-lane groups): lane i receives element
// (i % 4) of the 8-byte loads of source lanes i/4, 4 + i/4, 8 + i/4 and
// 12 + i/4.  With source lane s of group G reading row rb(G) + s/4,
// columns c0 + 4 (s % 4) .. +3, lane i of group G receives
//   T[rb(G) + 0..3][c0 + i].
__device__ __forceinline__ s16x4 tr_read4(const uint16_t *t, int row_base, int c0, int lane) {
  const int s = lane & 15;
  const uint16_t *p = t + swz(row_base + (s >> 2), c0 + 4 * (s & 3));
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<__attribute__((address_space(3))) s16x4 *>(
          reinterpret_cast<uintptr_t>(p)));
}

// MFMA operand (16 x 32 with K = rows) whose lane 16G + i holds the column
// c0 + i of rows ra(G) + 0..3 and rb(G) + 0..3.
template <class V8>
__device__ __forceinline__ V8 tr_operand(const uint16_t *t, int ra, int rb, int c0, int lane) {
  const s16x4 a = tr_read4(t, ra, c0, lane);
  const s16x4 b = tr_read4(t, rb, c0, lane);
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  return from_bits<V8>(make_uint4(ua.x, ua.y, ub.x, ub.y));
}

}  // namespace ssla
