// Row L2 normalisation (memory.py:30-31, 136-139) and the packing of the
// normalised sub-keys into the MFMA A-operand layout of score_select.hip.
#include "common.h"
#include "layout.h"

namespace mpl {

// 16 lanes per row, 16 rows per 256-thread block.
__global__ __launch_bounds__(256) void l2norm_kernel(const float* __restrict__ x, int64_t rows,
                                                     int dim, float eps, float* y,
                                                     _Float16* __restrict__ y16,
                                                     float* __restrict__ row_len) {
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  float s = 0.f;
  if (row < rows) {
    const float* xr = x + row * dim;
    for (int j = l; j < dim; j += 16) {
      float v = xr[j];
      s = fmaf(v, v, s);
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 16);
  if (row < rows) {
    const float tot = s + eps;
    const float r = 1.0f / sqrtf(tot);
    const float* xr = x + row * dim;
    float* yr = y + row * dim;
    _Float16* hr = y16 != nullptr ? y16 + row * dim : nullptr;
    for (int j = l; j < dim; j += 16) {
      const float v = xr[j] * r;
      yr[j] = v;
      if (hr != nullptr) hr[j] = (_Float16)v;
    }
    if (row_len != nullptr && l == 0) row_len[row] = sqrtf(tot) / sqrtf((float)dim);
  }
}

// One thread per 16-byte operand vector of the packed layout (layout.h).
template <typename T>
__global__ __launch_bounds__(256) void pack_keys_kernel(const float* __restrict__ khat, int HC, int n,
                                                        int half, int HP, int nblk,
                                                        uint4* __restrict__ packed) {
  const int vpl = KeyPack<T>::vectors_per_lane(HP);
  const int64_t total = (int64_t)HC * nblk * vpl * kWave;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const int lane = (int)(t % kWave);
  const int v = (int)((t / kWave) % vpl);
  const int blk = (int)((t / ((int64_t)kWave * vpl)) % nblk);
  const int hc = (int)(t / ((int64_t)kWave * vpl * nblk));
  const int key = blk * 32 + (lane & 31);
  float e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = 0.f;
  const int per = KeyPack<T>::elems_per_vector();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i < per) {
      const int dim = KeyPack<T>::dim_of(v, i, lane);
      if (key < n && dim < half) e[i] = khat[((int64_t)hc * n + key) * half + dim];
    }
  }
  packed[t] = KeyPack<T>::pack(e);
}

template <typename T>
static int pack_impl(const float* khat, int HC, int n, int half, void* packed, hipStream_t s) {
  const int HP = KeyPack<T>::padded_half(half);
  const int nblk = (int)cdiv(n, 32);
  const int64_t total = (int64_t)HC * nblk * KeyPack<T>::vectors_per_lane(HP) * kWave;
  pack_keys_kernel<T><<<(unsigned)cdiv(total, 256), 256, 0, s>>>(khat, HC, n, half, HP, nblk,
                                                                (uint4*)packed);
  return check_launch("mpl_pack_keys");
}

}  // namespace mpl

using namespace mpl;

extern "C" int mpl_l2_normalize(const float* x, int64_t rows, int dim, float eps, float* y,
                                void* y16, float* row_len, void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && dim > 0, MPL_EINVAL, "mpl_l2_normalize: bad sizes");
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(x && y, MPL_EINVAL, "mpl_l2_normalize: null buffer");
  l2norm_kernel<<<(unsigned)cdiv(rows, 16), 256, 0, (hipStream_t)stream>>>(x, rows, dim, eps, y,
                                                                             (_Float16*)y16, row_len);
  return check_launch("mpl_l2_normalize");
}

extern "C" size_t mpl_packed_keys_bytes(int H, int n, int half, int score_dtype) {
  if (H <= 0 || n <= 0 || half <= 0 || half > 128) return 0;
  const int64_t nblk = cdiv(n, 32);
  if (score_dtype == MPL_F16)
    return (size_t)(2 * H) * nblk * 32 * KeyPack<_Float16>::padded_half(half) * sizeof(_Float16);
  if (score_dtype == MPL_F32)
    return (size_t)(2 * H) * nblk * 32 * KeyPack<float>::padded_half(half) * sizeof(float);
  return 0;
}

extern "C" int mpl_pack_keys(const float* sub_keys, int H, int n, int half, int score_dtype,
                             float* keys_hat, void* packed, void* stream) {
  clear_error();
  MPL_REQUIRE(sub_keys && packed && H > 0 && n > 0 && half > 0, MPL_EINVAL,
              "mpl_pack_keys: bad arguments");
  MPL_REQUIRE(half <= 128, MPL_EUNSUPPORTED, "mpl_pack_keys: half=%d > 128", half);
  MPL_REQUIRE(score_dtype == MPL_F16 || score_dtype == MPL_F32, MPL_EINVAL,
              "mpl_pack_keys: score_dtype must be MPL_F16 or MPL_F32");
  hipStream_t s = (hipStream_t)stream;
  const int64_t rows = (int64_t)2 * H * n;
  float* khat = keys_hat;
  MPL_REQUIRE(khat != nullptr, MPL_EINVAL, "mpl_pack_keys: keys_hat buffer is required");
  l2norm_kernel<<<(unsigned)cdiv(rows, 16), 256, 0, s>>>(sub_keys, rows, half, 1e-6f, khat, nullptr, nullptr);
  int rc = check_launch("mpl_pack_keys(normalise)");
  if (rc) return rc;
  return score_dtype == MPL_F16 ? pack_impl<_Float16>(khat, 2 * H, n, half, packed, s)
                                : pack_impl<float>(khat, 2 * H, n, half, packed, s);
}
