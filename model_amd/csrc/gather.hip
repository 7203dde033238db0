// Value read: out[m] = sum over the H*k fetched rows of w * values[slot]
// (memory.py:179-193), without materialising the fetched rows.
//
// One wave per token.  Lane i < R loads the token's slot id and weight; rows
// are then broadcast from those lanes.  A row of d elements is LPR lanes x 16
// bytes; one wave-wide 128-bit load instruction covers RPI = 64 / LPR rows
// (for d = 256 fp16: 32 lanes per 512-byte row, two rows per instruction).
// Accumulation is fp32 per lane; lanes holding the same columns of different
// rows are summed with cross-lane shuffles at the end.
#include "common.h"

namespace mpl {

template <typename V>
struct Vec16;

template <>
struct Vec16<_Float16> {
  static constexpr int kElems = 8;
  __device__ static void unpack(uint4 u, float* f) {
    const half8 h = __builtin_bit_cast(half8, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)h[i];
  }
};

template <>
struct Vec16<float> {
  static constexpr int kElems = 4;
  __device__ static void unpack(uint4 u, float* f) {
    f[0] = __uint_as_float(u.x);
    f[1] = __uint_as_float(u.y);
    f[2] = __uint_as_float(u.z);
    f[3] = __uint_as_float(u.w);
  }
};

constexpr int kGatherThreads = 256;

// VR = 16-byte vectors per row.  Either VR divides 64 (several rows per
// instruction) or VR is a multiple of 64 (VR/64 vectors per lane per row).
template <typename V, int VR>
__global__ __launch_bounds__(kGatherThreads) void gather_wsum_kernel(
    const V* __restrict__ values, int64_t N, const int32_t* __restrict__ slots,
    const float* __restrict__ weights, int64_t M, int R, int shuffle, float* __restrict__ out) {
  constexpr int LPR = VR <= kWave ? VR : kWave;
  constexpr int RPI = kWave / LPR;
  constexpr int VPL = VR <= kWave ? 1 : VR / kWave;
  constexpr int VE = Vec16<V>::kElems;
  constexpr int NB = VPL >= 4 ? 4 : 16 / VPL;  // row groups in flight per lane
  const int64_t m = (int64_t)blockIdx.x * (kGatherThreads / kWave) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (m >= M) return;
  const int sub = lane / LPR;
  const int col = lane % LPR;
  float acc[VPL][VE];
#pragma unroll
  for (int v = 0; v < VPL; ++v)
#pragma unroll
    for (int e = 0; e < VE; ++e) acc[v][e] = 0.f;

  const uint4* base = (const uint4*)values;
  for (int r0 = 0; r0 < R; r0 += kWave) {
    const int rr = r0 + lane;
    const bool in = rr < R;
    int sl = slots[m * R + (in ? rr : 0)];  // unconditional (clamped) loads
    float ww = weights[m * R + (in ? rr : 0)];
    if (shuffle) sl = (int)(((int64_t)sl + N / 2 + 1) % N);
    sl = in ? (int)min(max((int64_t)sl, (int64_t)0), N - 1) : 0;  // out-of-range ids read the nearest row
    ww = in ? ww : 0.f;
    const int nr = min(kWave, R - r0);
    const int groups = (nr + RPI - 1) / RPI;  // row groups of this chunk
    // Batches of NB row groups: all NB loads are issued before any is used.
    for (int g0 = 0; g0 < groups; g0 += NB) {
      uint4 buf[NB][VPL];
      float wv[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const bool ok = g0 + b < groups;
        const int row = ok ? (g0 + b) * RPI + sub : 0;  // rows past nr carry weight 0 and slot 0
        const int s = __shfl(sl, row);
        const float w = __shfl(ww, row);
        wv[b] = ok ? w : 0.f;
        const uint4* src = base + (int64_t)s * VR + col;
#pragma unroll
        for (int v = 0; v < VPL; ++v) buf[b][v] = src[v * kWave];
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          float f[VE];
          Vec16<V>::unpack(buf[b][v], f);
#pragma unroll
          for (int e = 0; e < VE; ++e) acc[v][e] = fmaf(wv[b], f[e], acc[v][e]);
        }
      }
    }
  }
#pragma unroll
  for (int off = LPR; off < kWave; off <<= 1)
#pragma unroll
    for (int v = 0; v < VPL; ++v)
#pragma unroll
      for (int e = 0; e < VE; ++e) acc[v][e] += __shfl_xor(acc[v][e], off);
  if (sub == 0) {
    float* o = out + m * (int64_t)(VR * VE);
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      float4* dst = (float4*)(o + (v * kWave + col) * VE);
#pragma unroll
      for (int e = 0; e < VE; e += 4) dst[e / 4] = make_float4(acc[v][e], acc[v][e + 1], acc[v][e + 2], acc[v][e + 3]);
    }
  }
}

// Any d: one thread per (token, column).
template <typename V>
__global__ __launch_bounds__(256) void gather_wsum_generic(const V* __restrict__ values, int64_t N, int d,
                                                          const int32_t* __restrict__ slots,
                                                          const float* __restrict__ weights, int64_t M,
                                                          int R, int shuffle, float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M * d) return;
  const int64_t m = t / d;
  const int j = (int)(t % d);
  float acc = 0.f;
  for (int r = 0; r < R; ++r) {
    int64_t s = slots[m * R + r];
    if (shuffle) s = (s + N / 2 + 1) % N;
    s = s < 0 ? 0 : (s >= N ? N - 1 : s);
    acc = fmaf(weights[m * R + r], (float)values[s * d + j], acc);
  }
  out[t] = acc;
}

template <typename V>
static int gather_impl(const V* values, int64_t N, int d, const int32_t* slots, const float* w, int64_t M,
                       int R, int shuffle, float* out, hipStream_t s) {
  const int64_t bytes = (int64_t)d * sizeof(V);
  const unsigned blocks = (unsigned)cdiv(M, kGatherThreads / kWave);
  if (bytes % 16 == 0 && ((uintptr_t)values % 16) == 0 && ((uintptr_t)out % 16) == 0) {
    const int VR = (int)(bytes / 16);
    switch (VR) {
#define MPL_G(vr)                                                                                      \
  case vr:                                                                                             \
    gather_wsum_kernel<V, vr><<<blocks, kGatherThreads, 0, s>>>(values, N, slots, w, M, R, shuffle, out); \
    return check_launch("mpl_gather_wsum");
      MPL_G(1) MPL_G(2) MPL_G(4) MPL_G(8) MPL_G(16) MPL_G(32) MPL_G(64) MPL_G(128) MPL_G(256)
#undef MPL_G
      default: break;
    }
  }
  gather_wsum_generic<V><<<(unsigned)cdiv(M * d, 256), 256, 0, s>>>(values, N, d, slots, w, M, R, shuffle, out);
  return check_launch("mpl_gather_wsum(generic)");
}

}  // namespace mpl

using namespace mpl;

extern "C" int mpl_gather_wsum(const void* values, int values_dtype, int64_t N, int d, const int32_t* slots,
                               const float* weights, int64_t M, int R, int shuffle_reads, float* out,
                               void* stream) {
  clear_error();
  MPL_REQUIRE(N > 0 && d > 0 && M >= 0 && R > 0, MPL_EINVAL, "mpl_gather_wsum: bad sizes");
  if (M == 0) return MPL_OK;
  MPL_REQUIRE(values && slots && weights && out, MPL_EINVAL, "mpl_gather_wsum: null buffer");
  hipStream_t s = (hipStream_t)stream;
  if (values_dtype == MPL_F16)
    return gather_impl<_Float16>((const _Float16*)values, N, d, slots, weights, M, R, shuffle_reads, out, s);
  if (values_dtype == MPL_F32)
    return gather_impl<float>((const float*)values, N, d, slots, weights, M, R, shuffle_reads, out, s);
  set_error("mpl_gather_wsum: values_dtype must be MPL_F16 or MPL_F32");
  return MPL_EINVAL;
}
