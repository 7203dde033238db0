// Shared helpers for the gfx950 memory-layer lookup kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "../../include/mpl.h"

namespace mpl {

// Thread-local error message behind mpl_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Launch-status check shared by every entry point.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return MPL_EHIP;
  }
  return MPL_OK;
}

// Lanes l and l+32 exchange halves: with (a, b) the values of one register
// pair, lane l < 32 ends with (a[l], a[l+32]) and lane l >= 32 with
// (b[l-32], b[l]).  One v_permlane32_swap on gfx950.
__device__ inline void half_swap(float& a, float& b) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

}  // namespace mpl

#define MPL_REQUIRE(cond, code, ...)      \
  do {                                    \
    if (!(cond)) {                        \
      ::mpl::set_error(__VA_ARGS__);      \
      return (code);                      \
    }                                     \
  } while (0)
