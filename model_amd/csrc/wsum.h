// Weighted row sum of one token, shared by the value read (gather.hip) and
// the fused stage-2 + value read (score_select.hip): memory.py:184-193,
// out[m] = sum_r w[m,r] * values[slot[m,r]] without materialising the rows.
//
// One wave per token.  Lane i of a chunk holds row i's slot id and weight;
// rows are broadcast from those lanes.  A row of d elements is LPR lanes x 16
// bytes; one wave-wide 128-bit load instruction covers RPI = 64 / LPR rows
// (for d = 256 fp16: 32 lanes per 512-byte row, two rows per instruction).
// Accumulation is fp32 per lane; lanes holding the same columns of different
// rows are summed with cross-lane shuffles at the end.
#pragma once
#include "common.h"

namespace mpl {

// A 16-byte load marked non-temporal: with the hint the rows do not
// displace other lines in L2 and the Infinity Cache.  Which load a table's
// rows get depends on whether the table can stay in the 256 MB Infinity
// Cache between lookups:
//   - larger tables are streamed: a row is read once per lookup and not again
//     before it would be evicted, so the hint helps (4,096 tokens on the
//     34 GB table: 24.5 us per read non-temporal, 28.3 us plain);
//   - tables that fit are read again by the next lookup: ordinary loads keep
//     them resident (8,192 tokens on the 134 MB table: 39.4 us plain, 48.4 us
//     non-temporal, whose rows came from HBM every time).
// Both measured on MI355X, random 512-byte rows, rotating token batches.
typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_nt(const uint4* p) {
  const u32x4_nt v = __builtin_nontemporal_load((const u32x4_nt*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Value tables above this many bytes are read with non-temporal loads.
constexpr int64_t kStreamTableBytes = (int64_t)192 << 20;

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

// VR = 16-byte vectors per row.  Either VR divides 64 (several rows per
// instruction) or VR is a multiple of 64 (VR/64 vectors per lane per row).
//
// NBR = row groups per batch when a row group is one vector per lane.  The
// compiler schedules the loads of a batch itself: with NBR = 32 (the
// standalone read) it interleaves each load with the sums of the one before
// (about two in flight per wave) at low register use, which measured fastest
// at 4,096 tokens on the 34 GB table: 24.0 us per launch against 24.9-25.1 us
// with NBR = 16 and 26.2 us with all 32 loads forced ahead of the sums.  The
// fused stage-2 kernel keeps 16.  Batching never changes the order of the
// sums, so every NBR gives the same bits.
template <typename V, int VR, int NBR = 16, bool NT = true>
struct Wsum {
  static constexpr int LPR = VR <= kWave ? VR : kWave;
  static constexpr int RPI = kWave / LPR;
  static constexpr int VPL = VR <= kWave ? 1 : VR / kWave;
  static constexpr int VE = Vec16<V>::kElems;
  static constexpr int NB = VPL == 1 ? NBR : (VPL >= 4 ? 4 : 16 / VPL);  // row groups per batch
  float acc[VPL][VE];

  __device__ __forceinline__ Wsum() {
#pragma unroll
    for (int v = 0; v < VPL; ++v)
#pragma unroll
      for (int e = 0; e < VE; ++e) acc[v][e] = 0.f;
  }

  // Adds rows 0..nr-1 of a chunk (nr <= 64): lane i holds row i's slot id
  // `sl` (already in [0, N)) and weight `ww`.  Batches of NB row groups: all
  // NB loads are issued before any is used.
  __device__ __forceinline__ void add_chunk(const uint4* base, int sl, float ww, int nr, int lane) {
    const int sub = lane / LPR;
    const int col = lane % LPR;
    const int groups = (nr + RPI - 1) / RPI;
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
        for (int v = 0; v < VPL; ++v) buf[b][v] = NT ? load_nt(src + v * kWave) : src[v * kWave];
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

  // Adds one row group already loaded (VR <= 64: one vector per lane) with
  // its weight: the arithmetic add_chunk does for row group b, so a caller
  // adding groups 0, 1, ... in order gets add_chunk's bits.
  __device__ __forceinline__ void add_vec(uint4 u, float w) {
    static_assert(VPL == 1, "one vector per lane per row group");
    float f[VE];
    Vec16<V>::unpack(u, f);
#pragma unroll
    for (int e = 0; e < VE; ++e) acc[0][e] = fmaf(w, f[e], acc[0][e]);
  }

  // Sums the row groups across lanes and writes the token's d outputs.
  __device__ __forceinline__ void store(float* o, int lane) {
#pragma unroll
    for (int off = LPR; off < kWave; off <<= 1)
#pragma unroll
      for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[v][e] += __shfl_xor(acc[v][e], off);
    if (lane / LPR == 0) {
      const int col = lane % LPR;
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        float4* dst = (float4*)(o + (v * kWave + col) * VE);
#pragma unroll
        for (int e = 0; e < VE; e += 4) dst[e / 4] = make_float4(acc[v][e], acc[v][e + 1], acc[v][e + 2], acc[v][e + 3]);
      }
    }
  }
};

}  // namespace mpl
