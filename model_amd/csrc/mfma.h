// MFMA operand helpers shared by the scoring kernels (score_select.hip,
// balance.hip): the fp16 (v_mfma_f32_32x32x16_f16) and fp32
// (v_mfma_f32_32x32x2_f32) tiles, query operand loads, and LDS-DMA waits.
//
// Output layout of a 32x32 tile C = A . B (A rows i, B columns j): lane l
// holds column j = l % 32 and, in register r < 16, row
// i = 8*(r/4) + 4*(l/32) + r%4.
#pragma once

#include "common.h"

namespace mpl {

template <typename T>
struct Mfma;

template <>
struct Mfma<_Float16> {
  typedef half8 Op;
  __device__ static f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  // B operand for chunk c: dims 16c + 8*(lane/32) + [0,8) of fp16 query row
  // q (fp16 scoring requires half % 8 == 0, so this is one aligned 16-byte
  // load).  The load is unconditional and lanes out of range are zeroed by a
  // multiply with 0: a select of the loaded value is turned by the compiler
  // into a branch around the load with its own wait, which serialises the
  // chunks (one memory round trip each).  A lane out of range reads finite
  // data of its own row (or row 0), so the product is 0.
  __device__ static Op load_q(const _Float16* q, bool valid, int half, int c, int lane) {
    const int d0 = 16 * c + 8 * (lane >> 5);
    const Op o = *(const half8*)(q + (d0 < half ? d0 : 0));
    const _Float16 m = (valid && d0 < half) ? (_Float16)1.f : (_Float16)0.f;
    return o * m;
  }
  __device__ static Op from_vec(uint4 u, int) { return __builtin_bit_cast(half8, u); }
  // Raw fp32 query dims 16c + 8*(lane/32) + [0,8): two aligned 16-byte loads,
  // zeroed when out of range by a multiply with 0 (as in load_q); adds their
  // squares to ss.
  static constexpr int kQElems = 8;
  __device__ static void load_q_raw(const float* q, bool valid, int half, int c, int lane, float* x, float& ss) {
    const int d0 = 16 * c + 8 * (lane >> 5);
    const float m = (valid && d0 < half) ? 1.f : 0.f;
    const float4* src = (const float4*)(q + (d0 < half ? d0 : 0));
    const float4 u = src[0], v = src[1];
    x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
    x[4] = v.x; x[5] = v.y; x[6] = v.z; x[7] = v.w;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[i] *= m;
      ss = fmaf(x[i], x[i], ss);
    }
  }
  __device__ static Op scale_q(const float* x, float r) {
    Op o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (_Float16)(x[i] * r);
    return o;
  }
};

template <>
struct Mfma<float> {
  typedef float Op;
  __device__ static f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static Op load_q(const float* q, bool valid, int half, int c, int lane) {
    const int d = 2 * c + (lane >> 5);
    return q[min(d, half - 1)] * ((valid && d < half) ? 1.f : 0.f);
  }
  __device__ static Op from_vec(uint4 u, int e) {
    const unsigned w = e == 0 ? u.x : e == 1 ? u.y : e == 2 ? u.z : u.w;
    return __uint_as_float(w);
  }
  static constexpr int kQElems = 1;
  __device__ static void load_q_raw(const float* q, bool valid, int half, int c, int lane, float* x, float& ss) {
    const int d = 2 * c + (lane >> 5);
    x[0] = q[min(d, half - 1)] * ((valid && d < half) ? 1.f : 0.f);
    ss = fmaf(x[0], x[0], ss);
  }
  __device__ static Op scale_q(const float* x, float r) { return x[0] * r; }
};

// s_waitcnt that waits until at most N vector-memory loads of this wave are
// outstanding (gfx9 encoding; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt_le() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

typedef __attribute__((address_space(3))) void lds_void;

}  // namespace mpl
