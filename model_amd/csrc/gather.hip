// Value read: out[m] = sum over the H*k fetched rows of w * values[slot]
// (memory.py:179-193), without materialising the fetched rows.  One wave per
// token; the row sum itself is Wsum (wsum.h), shared with the fused stage-2
// kernel of score_select.hip.
#include "common.h"
#include "wsum.h"

namespace mpl {

constexpr int kGatherThreads = 256;

template <typename V, int VR, bool NT>
__global__ __launch_bounds__(kGatherThreads) void gather_wsum_kernel(
    const V* __restrict__ values, int64_t N, const int32_t* __restrict__ slots,
    const float* __restrict__ weights, int64_t M, int R, int shuffle, float* __restrict__ out) {
  const int64_t m = (int64_t)blockIdx.x * (kGatherThreads / kWave) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (m >= M) return;
  Wsum<V, VR, 32, NT> acc;
  const uint4* base = (const uint4*)values;
  for (int r0 = 0; r0 < R; r0 += kWave) {
    const int rr = r0 + lane;
    const bool in = rr < R;
    int sl = slots[m * R + (in ? rr : 0)];  // unconditional (clamped) loads
    float ww = weights[m * R + (in ? rr : 0)];
    if (shuffle) sl = (int)(((int64_t)sl + N / 2 + 1) % N);
    sl = in ? (int)min(max((int64_t)sl, (int64_t)0), N - 1) : 0;  // out-of-range ids read the nearest row
    ww = in ? ww : 0.f;
    acc.add_chunk(base, sl, ww, min(kWave, R - r0), lane);
  }
  acc.store(out + m * (int64_t)(VR * Vec16<V>::kElems), lane);
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
    const bool nt = N * bytes > kStreamTableBytes;
    switch (VR) {
#define MPL_G(vr)                                                                                              \
  case vr:                                                                                                     \
    if (nt)                                                                                                    \
      gather_wsum_kernel<V, vr, true><<<blocks, kGatherThreads, 0, s>>>(values, N, slots, w, M, R, shuffle, out); \
    else                                                                                                       \
      gather_wsum_kernel<V, vr, false><<<blocks, kGatherThreads, 0, s>>>(values, N, slots, w, M, R, shuffle, out); \
    return check_launch("mpl_gather_wsum");
      MPL_G(1) MPL_G(2) MPL_G(4) MPL_G(8) MPL_G(16) MPL_G(32) MPL_G(64) MPL_G(128) MPL_G(256)
#undef MPL_G
      default: break;
    }
  }
  gather_wsum_generic<V><<<(unsigned)cdiv(M * d, 256), 256, 0, s>>>(values, N, d, slots, w, M, R, shuffle, out);
  return check_launch("mpl_gather_wsum(generic)");
}

// Row copy for the host tier: out[i] = table[clamp(idx[i])] for i < rows,
// rows = min(count, *count_dev) (count_dev may be null).  The table may be
// device memory or pinned host memory mapped for the device, in which case
// every 16-byte vector crosses the bus once; kUnroll vectors per thread are
// loaded before any is stored, so several reads are in flight per lane.
constexpr int kRowCopyUnroll = 4;

template <int W>
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint32_t* __restrict__ table, int64_t N, int wpr,
                                                          const int32_t* __restrict__ idx, int64_t count,
                                                          const int32_t* __restrict__ count_dev,
                                                          uint32_t* __restrict__ out) {
  // W 32-bit words per access (4: 16-byte vectors); wpr accesses per row
  typedef uint32_t Acc __attribute__((ext_vector_type(W)));
  const int64_t rows = count_dev != nullptr ? min(count, (int64_t)*count_dev) : count;
  const int64_t total = rows * wpr;
  const int64_t stride = (int64_t)gridDim.x * 256 * kRowCopyUnroll;
  for (int64_t t0 = (int64_t)blockIdx.x * 256 * kRowCopyUnroll + threadIdx.x; t0 < total; t0 += stride) {
    Acc v[kRowCopyUnroll];
    int64_t dst[kRowCopyUnroll];
#pragma unroll
    for (int u = 0; u < kRowCopyUnroll; ++u) {
      const int64_t t = t0 + (int64_t)u * 256;
      const bool ok = t < total;
      const int64_t r = ok ? t / wpr : 0;
      const int c = ok ? (int)(t - r * wpr) : 0;
      int64_t sl = idx[r];
      sl = sl < 0 ? 0 : (sl >= N ? N - 1 : sl);
      v[u] = ((const Acc*)table)[sl * wpr + c];
      dst[u] = ok ? t : -1;
    }
#pragma unroll
    for (int u = 0; u < kRowCopyUnroll; ++u)
      if (dst[u] >= 0) ((Acc*)out)[dst[u]] = v[u];
  }
}

}  // namespace mpl

using namespace mpl;

extern "C" int mpl_gather_rows(const void* table, int dtype, int64_t N, int d, const int32_t* idx, int64_t count,
                               const int32_t* count_dev, void* out, void* stream) {
  clear_error();
  MPL_REQUIRE(N > 0 && d > 0 && count >= 0, MPL_EINVAL, "mpl_gather_rows: bad sizes N=%lld d=%d count=%lld",
              (long long)N, d, (long long)count);
  MPL_REQUIRE(dtype == MPL_F16 || dtype == MPL_F32, MPL_EINVAL, "mpl_gather_rows: dtype must be MPL_F16 or MPL_F32");
  if (count == 0) return MPL_OK;
  MPL_REQUIRE(table && idx && out, MPL_EINVAL, "mpl_gather_rows: null buffer");
  const int64_t row_bytes = (int64_t)d * (dtype == MPL_F16 ? 2 : 4);
  MPL_REQUIRE(row_bytes % 4 == 0, MPL_EUNSUPPORTED, "mpl_gather_rows: rows of %lld bytes (need a multiple of 4)",
              (long long)row_bytes);
  hipStream_t s = (hipStream_t)stream;
  const bool vec = row_bytes % 16 == 0 && ((uintptr_t)table % 16) == 0 && ((uintptr_t)out % 16) == 0;
  const int wpr = (int)(vec ? row_bytes / 16 : row_bytes / 4);
  const int64_t work = cdiv(count * wpr, 256 * kRowCopyUnroll);
  const unsigned blocks = (unsigned)(work < 4096 ? (work > 0 ? work : 1) : 4096);
  if (vec)
    gather_rows_kernel<4><<<blocks, 256, 0, s>>>((const uint32_t*)table, N, wpr, idx, count, count_dev,
                                                 (uint32_t*)out);
  else
    gather_rows_kernel<1><<<blocks, 256, 0, s>>>((const uint32_t*)table, N, wpr, idx, count, count_dev,
                                                 (uint32_t*)out);
  return check_launch("mpl_gather_rows");
}

extern "C" int mpl_host_device_pointer(void* host_ptr, void** dev_ptr) {
  clear_error();
  MPL_REQUIRE(host_ptr && dev_ptr, MPL_EINVAL, "mpl_host_device_pointer: null argument");
  void* p = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&p, host_ptr, 0);
  // the failed query is reported here; clear HIP's sticky per-thread error,
  // or the caller's next launch check would report it again
  if (e != hipSuccess) (void)hipGetLastError();
  MPL_REQUIRE(e == hipSuccess && p != nullptr, MPL_EINVAL,
              "mpl_host_device_pointer: %p is not pinned host memory mapped for the device (%s)", host_ptr,
              hipGetErrorString(e));
  *dev_ptr = p;
  return MPL_OK;
}

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
