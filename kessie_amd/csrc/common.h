// Shared device/host helpers for the gfx950 KeSSie kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

#include "../../include/kessie_mi355x.h"

namespace kessie {

// ---------------------------------------------------------------------------
// Error state (thread-local, host side)
// ---------------------------------------------------------------------------
void set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
int last_status();

// Records a HIP launch/runtime failure; returns KESSIE_ERR_HIP or KESSIE_OK.
int check_launch(const char* what);

#define KESSIE_REQUIRE(cond, code, ...)          \
  do {                                           \
    if (!(cond)) {                               \
      ::kessie::set_error((code), __VA_ARGS__);  \
      return (code);                             \
    }                                            \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int dtype_size(int dtype) {
  switch (dtype) {
    case KESSIE_DTYPE_F32: return 4;
    case KESSIE_DTYPE_BF16: return 2;
    case KESSIE_DTYPE_F16: return 2;
    default: return 0;
  }
}

// ---------------------------------------------------------------------------
// Element conversions.  bf16 <-> f32 use the hardware's round-to-nearest-even
// conversion (v_cvt_pk_bf16_f32 on gfx950), the rounding torch uses.
// ---------------------------------------------------------------------------
typedef __bf16 bf16_t;
typedef _Float16 f16_t;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(f16_t x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return static_cast<bf16_t>(x); }
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return static_cast<f16_t>(x); }

// bf16 bit pattern -> f32 (exact).
__device__ __forceinline__ float bf16_lo_to_f32(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16_hi_to_f32(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }

// ---------------------------------------------------------------------------
// Vector types
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__host__ __device__ __forceinline__ int div_up(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ __forceinline__ int64_t div_up(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace kessie
