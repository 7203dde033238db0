// Packed sub-key layout shared by normalize.hip (writer) and score_select.hip
// (reader).
//
// The scoring kernel computes S^T = K . Q^T with 32x32 MFMA tiles: keys are
// the A operand (rows), queries the B operand (columns).  For each codebook
// hc = h*2 + c and each block of 32 keys the packed buffer holds, for every
// lane of a wave, the A-operand registers that lane needs, as consecutive
// 16-byte vectors:  packed[hc][blk][v][lane] (uint4).  A wave therefore reads
// one key block with fully coalesced, bank-conflict-free 16-byte accesses.
//
//   fp16 (v_mfma_f32_32x32x16_f16): chunk c = v covers dims [16c, 16c+16);
//        lane l holds key (l % 32), dims 16c + 8*(l/32) + [0, 8).
//   fp32 (v_mfma_f32_32x32x2_f32):  vector v holds chunks 4v..4v+3; chunk c
//        covers dims [2c, 2c+2); lane l holds key (l % 32), dim 2c + l/32.
//
// The B operand (queries) uses the same lane -> dim map, so the MFMA's K
// reduction pairs equal dims whatever the hardware's K order is.  `half` is
// zero-padded to HP (a power of two) and n to a multiple of 32.
#pragma once

#include "common.h"

namespace mpl {

template <typename T>
struct KeyPack;

template <>
struct KeyPack<_Float16> {
  static constexpr int kChunk = 16;  // dims per MFMA
  static constexpr int kOpsPerVec = 1;
  static constexpr bool kContiguous = true;  // a lane's dims of a vector are consecutive
  __host__ __device__ static int padded_half(int half) {
    return half <= 16 ? 16 : half <= 32 ? 32 : half <= 64 ? 64 : 128;
  }
  __host__ __device__ static constexpr int vectors_per_lane(int HP) { return HP / 16; }
  __device__ static constexpr int elems_per_vector() { return 8; }
  __device__ static int dim_of(int v, int i, int lane) { return 16 * v + 8 * (lane >> 5) + i; }
  __device__ static uint4 pack(const float* e) {
    half8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16)e[i];
    return __builtin_bit_cast(uint4, h);
  }
};

template <>
struct KeyPack<float> {
  static constexpr int kChunk = 2;
  static constexpr int kOpsPerVec = 4;
  static constexpr bool kContiguous = false;
  __host__ __device__ static int padded_half(int half) {
    return half <= 8 ? 8 : half <= 16 ? 16 : half <= 32 ? 32 : half <= 64 ? 64 : 128;
  }
  __host__ __device__ static constexpr int vectors_per_lane(int HP) { return HP / 8; }
  __device__ static constexpr int elems_per_vector() { return 4; }
  __device__ static int dim_of(int v, int i, int lane) { return 8 * v + 2 * i + (lane >> 5); }
  __device__ static uint4 pack(const float* e) {
    uint4 u;
    u.x = __float_as_uint(e[0]);
    u.y = __float_as_uint(e[1]);
    u.z = __float_as_uint(e[2]);
    u.w = __float_as_uint(e[3]);
    return u;
  }
};

}  // namespace mpl
