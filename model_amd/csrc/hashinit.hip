// Hash-defined normal tables: element (row, col) of a [rows, cols] table is
//   index = row * cols + col                       (uint64, wrapping)
//   h     = splitmix64(splitmix64(seed) ^ index)
//   u1    = ((h >> 40) + 1) / 2^24                 in (0, 1]
//   u2    = (h & 0xFFFFFF) / 2^24                  in [0, 1)
//   z     = sqrt(-2 ln u1) cos(2 pi u2)            (Box-Muller, fp64)
//   value = (dtype)(float)(z * scale)              (fp64 -> fp32 -> dtype,
//                                                   round to nearest even)
// splitmix64 is the finalizer of Steele, Lea & Flood's SplitMix64 generator
// (OOPSLA 2014): x += 0x9E3779B97F4A7C15, then two xor-shift-multiply rounds
// and a final xor-shift.  Every element depends only on (seed, row, col), so a
// table far larger than host memory can be filled in place on the GPU while
// the CPU regenerates any subset of its rows with the same definition
// (oracle/hashinit.py is the numpy statement of it).  The memory pool's own
// init (memory.py:104-109) draws from jax.random.normal; this generator is
// for synthetic benchmark tables of the pool's shapes.
#include <math.h>

#include "common.h"

namespace mpl {
namespace {

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <typename V>
__global__ __launch_bounds__(256) void hash_fill_kernel(V* __restrict__ out, int64_t rows, int cols, uint64_t key,
                                                        double scale, int64_t row0) {
  const int64_t total = rows * (int64_t)cols;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / cols;
    const int64_t c = i - r * cols;
    const uint64_t index = (uint64_t)(row0 + r) * (uint64_t)cols + (uint64_t)c;
    const uint64_t h = splitmix64(key ^ index);
    const double u1 = (double)((h >> 40) + 1ull) * 0x1p-24;
    const double u2 = (double)(h & 0xFFFFFFull) * 0x1p-24;
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    // the fp32 value is materialised before the conversion to V: without the
    // barrier the compiler folds the two roundings into one double -> fp16
    // rounding, which differs from the definition wherever the fp32 value is
    // an fp16 tie (76 of 1,048,576 elements of a pool table)
    float f = (float)(z * scale);
    asm volatile("" : "+v"(f));
    out[i] = (V)f;
  }
}

}  // namespace
}  // namespace mpl

using namespace mpl;

extern "C" int mpl_hash_normal_fill(void* out, int dtype, int64_t rows, int cols, uint64_t seed, float scale,
                                    int64_t row0, void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && cols >= 1 && row0 >= 0, MPL_EINVAL,
              "mpl_hash_normal_fill: bad sizes rows=%lld cols=%d row0=%lld", (long long)rows, cols,
              (long long)row0);
  MPL_REQUIRE(dtype == MPL_F16 || dtype == MPL_F32, MPL_EINVAL, "mpl_hash_normal_fill: dtype must be MPL_F16 or MPL_F32");
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(out != nullptr, MPL_EINVAL, "mpl_hash_normal_fill: null output");
  hipStream_t s = (hipStream_t)stream;
  const uint64_t key = splitmix64(seed);
  const int64_t total = rows * (int64_t)cols;
  const unsigned grid = (unsigned)std::min<int64_t>(cdiv(total, 256), 65536);
  if (dtype == MPL_F16)
    hash_fill_kernel<_Float16><<<grid, 256, 0, s>>>((_Float16*)out, rows, cols, key, (double)scale, row0);
  else
    hash_fill_kernel<float><<<grid, 256, 0, s>>>((float*)out, rows, cols, key, (double)scale, row0);
  return check_launch("mpl_hash_normal_fill");
}
