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

// Backward of l2norm_kernel: dx = (dy - y (y . dy)) / sqrt(sum x^2 + eps),
// y = x / sqrt(sum x^2 + eps), times *scale when given.  16 lanes per row.
__global__ __launch_bounds__(256) void l2norm_bwd_kernel(const float* __restrict__ x, const float* __restrict__ dy,
                                                         int64_t rows, int dim, float eps,
                                                         const float* __restrict__ scale, float* __restrict__ dx) {
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  const int64_t rc = row < rows ? row : 0;
  const float* xr = x + rc * dim;
  const float* gr = dy + rc * dim;
  float ss = 0.f, xg = 0.f;
  for (int j = l; j < dim; j += 16) {
    const float v = xr[j], g = gr[j];
    ss = fmaf(v, v, ss);
    xg = fmaf(v, g, xg);
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) {
    ss += __shfl_xor(ss, o, 16);
    xg += __shfl_xor(xg, o, 16);
  }
  if (row >= rows) return;
  const float r = 1.0f / sqrtf(ss + eps);
  const float yg = xg * r;  // y . dy
  const float sc = scale != nullptr ? *scale : 1.f;
  float* dr = dx + row * dim;
  for (int j = l; j < dim; j += 16) dr[j] = sc * r * (gr[j] - xr[j] * r * yg);
}

// Normalise and pack in one pass: one wave per (codebook, block of 32 keys).
// Lane l owns exactly the dims of key l % 32 that the packed layout gives it
// (the other half sits in lane l ^ 32), so one half-swap completes the row's
// sum of squares and every lane writes its own operand vectors.
// With few key blocks (small n) the VPL vectors of a block are spread over
// `parts` waves (each recomputes the row norms and writes VPL / parts
// vectors) so that the launch still fills the GPU.
template <typename T, int VPL>
__global__ __launch_bounds__(256) void norm_pack_kernel(const float* __restrict__ keys, int HC, int n, int half,
                                                        int nblk, int parts, float* __restrict__ khat,
                                                        uint4* __restrict__ packed) {
  constexpr int PER = KeyPack<T>::elems_per_vector();
  const int64_t w = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (w >= (int64_t)HC * nblk * parts) return;  // wave-uniform
  const int part = (int)(w % parts);
  const int hc = (int)(w / parts / nblk), blk = (int)(w / parts % nblk);
  const int v0 = part * (VPL / parts), v1 = v0 + VPL / parts;
  const int key = blk * 32 + (lane & 31);
  const bool kin = key < n;
  const float* row = keys + ((int64_t)hc * n + (kin ? key : 0)) * half;
  float e[VPL][PER];
  float ss = 0.f;
  if (KeyPack<T>::kContiguous && (half & 7) == 0) {
    // fp16 packing: the lane's dims of vector v are 8 consecutive floats
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int d0 = KeyPack<T>::dim_of(v, 0, lane);
      const float4* src = (const float4*)(row + (d0 < half ? d0 : 0));  // clamped load, zeroed after
      const float4 a = src[0], b = src[1];
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        e[v][i] = (kin && d0 < half) ? x[i < 8 ? i : 0] : 0.f;
        ss = fmaf(e[v][i], e[v][i], ss);
      }
    }
  } else {
#pragma unroll
    for (int v = 0; v < VPL; ++v)
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int dim = KeyPack<T>::dim_of(v, i, lane);
        const float x = row[dim < half ? dim : 0];  // clamped load, zeroed after
        e[v][i] = (kin && dim < half) ? x : 0.f;
        ss = fmaf(e[v][i], e[v][i], ss);
      }
  }
  float a = ss, b = ss;
  half_swap(a, b);
  const float r = 1.0f / sqrtf(ss + ((lane >> 5) ? a : b) + 1e-6f);
  uint4* dst = packed + ((int64_t)hc * nblk + blk) * VPL * kWave;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    if (v < v0 || v >= v1) continue;
#pragma unroll
    for (int i = 0; i < PER; ++i) e[v][i] *= r;
    dst[v * kWave + lane] = KeyPack<T>::pack(e[v]);
  }
  if (khat != nullptr && kin) {
    float* kr = khat + ((int64_t)hc * n + key) * half;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      if (v < v0 || v >= v1) continue;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int dim = KeyPack<T>::dim_of(v, i, lane);
        if (dim < half) kr[dim] = e[v][i];
      }
    }
  }
}


// memory.py:143-146: T = exp(clip(log_t, ln min, ln max)), one thread (a
// NaN log_t stays NaN, as jnp.clip passes it).
__global__ void temperature_kernel(const float* __restrict__ log_t, float lo, float hi, float* __restrict__ t) {
  const float x = *log_t;
  t[0] = expf(x != x ? x : fminf(fmaxf(x, lo), hi));
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

extern "C" int mpl_temperature(const float* log_t, float log_min, float log_max, float* t, void* stream) {
  clear_error();
  MPL_REQUIRE(log_t != nullptr && t != nullptr, MPL_EINVAL, "mpl_temperature: null buffer");
  MPL_REQUIRE(log_min <= log_max, MPL_EINVAL, "mpl_temperature: log_min > log_max");
  temperature_kernel<<<1, 64, 0, (hipStream_t)stream>>>(log_t, log_min, log_max, t);
  return check_launch("mpl_temperature");
}

extern "C" int mpl_l2_normalize_bwd(const float* x, const float* dy, int64_t rows, int dim, float eps,
                                    const float* scale, float* dx, void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && dim > 0, MPL_EINVAL, "mpl_l2_normalize_bwd: bad sizes");
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(x && dy && dx, MPL_EINVAL, "mpl_l2_normalize_bwd: null buffer");
  l2norm_bwd_kernel<<<(unsigned)cdiv(rows, 16), 256, 0, (hipStream_t)stream>>>(x, dy, rows, dim, eps, scale, dx);
  return check_launch("mpl_l2_normalize_bwd");
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
  const int HC = 2 * H;
  const int nblk = (int)cdiv(n, 32);
  const int vpl = score_dtype == MPL_F16 ? KeyPack<_Float16>::vectors_per_lane(KeyPack<_Float16>::padded_half(half))
                                        : KeyPack<float>::vectors_per_lane(KeyPack<float>::padded_half(half));
  int parts = 1;  // aim for >= 1024 waves
  while (parts < vpl && (int64_t)HC * nblk * parts < 1024) parts *= 2;
  const unsigned blocks = (unsigned)cdiv((int64_t)HC * nblk * parts, 256 / kWave);
#define MPL_NP(T, V)                                                                                  \
  norm_pack_kernel<T, V><<<blocks, 256, 0, s>>>(sub_keys, HC, n, half, nblk, parts, keys_hat, (uint4*)packed)
  switch (vpl) {
    case 1: if (score_dtype == MPL_F16) MPL_NP(_Float16, 1); else MPL_NP(float, 1); break;
    case 2: if (score_dtype == MPL_F16) MPL_NP(_Float16, 2); else MPL_NP(float, 2); break;
    case 4: if (score_dtype == MPL_F16) MPL_NP(_Float16, 4); else MPL_NP(float, 4); break;
    case 8: if (score_dtype == MPL_F16) MPL_NP(_Float16, 8); else MPL_NP(float, 8); break;
    default: MPL_NP(float, 16); break;  // fp32 packing of half = 128
  }
#undef MPL_NP
  return check_launch("mpl_pack_keys");
}
