// Gumbel(0, 1) routing noise (memory.py:155-159: jax.random.gumbel over the
// score shape [M, H, 2, n], then select = score + routing_noise *
// noise_scale * gumbel).
//
// The reference draws it from JAX's key-split PRNG; this library fills the
// same [rows, n] fp32 tensor in one pass from a counter-based hash, so any
// element can be regenerated from (seed, row, j) alone:
//
//   a  = fmix32(lo32(row) ^ lo32(seed))
//   rk = fmix32(a ^ hi32(seed) ^ hi32(row))           (per-row key)
//   h  = fmix32(rk + j)                               (j < n)
//   u  = max((h >> 9) * 2^-23, FLT_MIN)               (JAX's uniform grid on [tiny, 1))
//   g  = -log(-log(u))
//
// fmix32 is the 32-bit finalizer of MurmurHash3 (Appleby; public domain): a
// bijection on 32-bit words.  u takes JAX's values: 23-bit multiples of
// 2^-23 below 1, clamped below at the smallest normal float, so g lies in
// [-4.47, 15.9] like jax.random.gumbel's.  The inner log is the accurate
// (ocml) logf: -log(u) near u = 1 is a small number whose relative precision
// the outer log needs.  The outer log is the hardware log2 times ln 2, whose
// error is absolute near its zero (e = 1) and relative elsewhere.
#include <float.h>
#include <math.h>

#include "common.h"

namespace mpl {

__device__ __forceinline__ uint32_t fmix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85ebca6bu;
  x ^= x >> 13;
  x *= 0xc2b2ae35u;
  x ^= x >> 16;
  return x;
}

__device__ __forceinline__ float gumbel_of(uint32_t rk, int j) {
  const uint32_t h = fmix32(rk + (uint32_t)j);
  const float u = fmaxf((float)(h >> 9) * 0x1p-23f, FLT_MIN);
  // e = -log(u) lies in [2^-23, 87.4]; near u = 1 it is small and the outer
  // log needs its relative precision, so it takes the accurate logf.  The
  // outer log only needs absolute precision where its result is near 0
  // (e near 1), which the hardware log2 gives: ln 2 * log2(e).
  const float e = -logf(u);
  return -0x1.62e43p-1f * __builtin_amdgcn_logf(e);
}

// One thread per four consecutive elements of a row.
__global__ __launch_bounds__(256) void gumbel_kernel(uint64_t seed, int64_t rows, int n, int n4, int vec,
                                                     float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * n4) return;
  const int64_t row = t / n4;
  const int j0 = (int)(t - row * n4) * 4;
  const uint32_t a = fmix32((uint32_t)row ^ (uint32_t)seed);
  const uint32_t rk = fmix32(a ^ (uint32_t)(seed >> 32) ^ (uint32_t)((uint64_t)row >> 32));
  float* o = out + row * n + j0;
  if (vec) {  // n % 4 == 0 and out 16-byte aligned: j0 + 3 < n
    *(float4*)o = make_float4(gumbel_of(rk, j0), gumbel_of(rk, j0 + 1), gumbel_of(rk, j0 + 2), gumbel_of(rk, j0 + 3));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (j0 + i < n) o[i] = gumbel_of(rk, j0 + i);
  }
}

}  // namespace mpl

using namespace mpl;

extern "C" int mpl_gumbel_noise(uint64_t seed, int64_t rows, int n, float* out, void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && n > 0, MPL_EINVAL, "mpl_gumbel_noise: bad sizes rows=%lld n=%d", (long long)rows, n);
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(out != nullptr, MPL_EINVAL, "mpl_gumbel_noise: null output");
  const int n4 = (n + 3) / 4;
  const int64_t threads = rows * n4;
  MPL_REQUIRE(cdiv(threads, 256) < ((int64_t)1 << 31), MPL_EUNSUPPORTED, "mpl_gumbel_noise: %lld rows too many",
              (long long)rows);
  const int vec = n % 4 == 0 && ((uintptr_t)out & 15) == 0;
  gumbel_kernel<<<(unsigned)cdiv(threads, 256), 256, 0, (hipStream_t)stream>>>(seed, rows, n, n4, vec, out);
  return check_launch("mpl_gumbel_noise");
}
