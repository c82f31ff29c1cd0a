// Shared helpers for the gfx950 kernels of libssla_amd.so.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>
#include <algorithm>

#include "../../include/ssla_amd.h"

namespace ssla {

// ---------------------------------------------------------------- errors --
void set_error(const char *fmt, ...);
void clear_error();

#define SSLA_CHECK_ARG(cond, ...)            \
  do {                                       \
    if (!(cond)) {                           \
      ::ssla::set_error(__VA_ARGS__);        \
      return SSLA_ERR_ARG;                   \
    }                                        \
  } while (0)

// Copy `bytes` (at most 4096) of device memory to host memory and wait for
// the stream: one copy into a per-thread pinned staging buffer (a pageable
// destination makes the runtime stage and synchronise each copy itself).
// Returns the HIP error.
hipError_t read_to_host(void *dst, const void *src, size_t bytes, hipStream_t st);

inline int launch_status(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return SSLA_ERR_LAUNCH;
  }
  return SSLA_OK;
}

inline bool aligned(const void *p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// --------------------------------------------------------------- vectors --
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;

// --------------------------------------------------------- element types --
// Raw 16-bit storage <-> fp32.  bf16 -> fp32 is an exact shift; fp32 -> bf16
// rounds to nearest-even (NaN kept quiet).
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT> struct Elem;
template <> struct Elem<SSLA_F32> {
  typedef float T;
  static __device__ __forceinline__ float load(const void *p, int64_t i) {
    return static_cast<const float *>(p)[i];
  }
  static __device__ __forceinline__ void store(void *p, int64_t i, float x) {
    static_cast<float *>(p)[i] = x;
  }
};
template <> struct Elem<SSLA_BF16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const void *p, int64_t i) {
    return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  }
  static __device__ __forceinline__ void store(void *p, int64_t i, float x) {
    static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(x);
  }
};
template <> struct Elem<SSLA_F16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const void *p, int64_t i) {
    return f16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  }
  static __device__ __forceinline__ void store(void *p, int64_t i, float x) {
    static_cast<uint16_t *>(p)[i] = f32_to_f16_bits(x);
  }
};

// exp2 on the hardware transcendental unit (v_exp_f32: relative error
// ~1 ulp over the normal range, flushes results below 2^-126 to 0).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ------------------------------------------------------------------- DPP --
// Shift right by N lanes inside each 16-lane DPP row; lanes whose source
// lies outside the row read 0 (bound_ctrl), so an add of the result folds
// into a single v_add_f32 with a DPP source.
template <int N>
__device__ __forceinline__ float row_shr(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, x), 0x110 + N, 0xf, 0xf, true));
}

// Inclusive prefix sum across the 16 lanes of each DPP row.
__device__ __forceinline__ float row_inclusive_scan(float x) {
  x += row_shr<1>(x);
  x += row_shr<2>(x);
  x += row_shr<4>(x);
  x += row_shr<8>(x);
  return x;
}

}  // namespace ssla
