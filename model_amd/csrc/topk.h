// Exact top-k building blocks on 64-bit keys.
//
// A candidate (score, index) is packed as
//     key = (orderable(score) << 32) | (0xFFFFFFFF - index)
// so that unsigned key order is (score descending, index ascending): the
// order of lax.top_k, ties going to the lowest index.  Key 0 is below every
// real candidate and marks an empty slot.
//
// TopList<KMAX> keeps the best KMAX keys sorted descending in registers.
// Candidates are merged in chunks of 8: an optimal 19-comparator network
// sorts the chunk, the bitonic split R[i] = max(A[i], B[KMAX-1-i]) keeps the
// KMAX best of both, and a bitonic merger re-sorts them (4 or 5 stages).
// An optional float payload travels with each key.
#pragma once

#include "common.h"

namespace mpl {

typedef unsigned long long u64;

__device__ __forceinline__ uint32_t orderable(float f) {
  const uint32_t b = __float_as_uint(f + 0.0f);  // -0 -> +0
  return b ^ ((b & 0x80000000u) ? 0xFFFFFFFFu : 0x80000000u);
}

__device__ __forceinline__ float from_orderable(uint32_t u) {
  const uint32_t b = (u & 0x80000000u) ? (u ^ 0x80000000u) : ~u;
  return __uint_as_float(b);
}

__device__ __forceinline__ u64 make_key(float s, int idx) {
  return ((u64)orderable(s) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ float key_score(u64 k) { return from_orderable((uint32_t)(k >> 32)); }
__device__ __forceinline__ int key_index(u64 k) { return (int)(0xFFFFFFFFu - (uint32_t)k); }

// Compare-exchange, larger key to `a`.
template <bool PAY>
__device__ __forceinline__ void cex(u64& a, u64& b, float& pa, float& pb) {
  const bool sw = a < b;
  const u64 t = sw ? b : a;
  b = sw ? a : b;
  a = t;
  if (PAY) {
    const float q = sw ? pb : pa;
    pb = sw ? pa : pb;
    pa = q;
  }
}

// Sorts 8 keys descending (optimal 19-comparator network).
template <bool PAY>
__device__ __forceinline__ void sort8(u64* c, float* p) {
#define MPL_CE(i, j) cex<PAY>(c[i], c[j], p[PAY ? i : 0], p[PAY ? j : 0])
  MPL_CE(0, 2); MPL_CE(1, 3); MPL_CE(4, 6); MPL_CE(5, 7);
  MPL_CE(0, 4); MPL_CE(1, 5); MPL_CE(2, 6); MPL_CE(3, 7);
  MPL_CE(0, 1); MPL_CE(2, 3); MPL_CE(4, 5); MPL_CE(6, 7);
  MPL_CE(2, 4); MPL_CE(3, 5);
  MPL_CE(1, 4); MPL_CE(3, 6);
  MPL_CE(1, 2); MPL_CE(3, 4); MPL_CE(5, 6);
#undef MPL_CE
}

template <int KMAX, bool PAY>
struct TopList {
  u64 key[KMAX];
  float pay[PAY ? KMAX : 1];

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) key[j] = 0;
#pragma unroll
    for (int j = 0; j < (PAY ? KMAX : 1); ++j) pay[j] = 0.f;
  }

  // Merge a sorted (descending) run of CN <= KMAX keys.
  template <int CN>
  __device__ __forceinline__ void merge(const u64* c, const float* cp) {
#pragma unroll
    for (int i = KMAX - CN; i < KMAX; ++i) {
      const u64 b = c[KMAX - 1 - i];
      const bool take = b > key[i];
      key[i] = take ? b : key[i];
      if (PAY) pay[PAY ? i : 0] = take ? cp[PAY ? KMAX - 1 - i : 0] : pay[PAY ? i : 0];
    }
    // Affine stage counter: every index below is a compile-time constant,
    // so the list stays in registers.
    constexpr int kStages = KMAX == 32 ? 5 : 4;
#pragma unroll
    for (int st = 0; st < kStages; ++st) {
      const int s = (KMAX / 2) >> st;
#pragma unroll
      for (int i = 0; i < KMAX; ++i) {
        if ((i & s) == 0) cex<PAY>(key[i], key[i + s], pay[PAY ? i : 0], pay[PAY ? i + s : 0]);
      }
    }
  }

  // Key at runtime position r (< KMAX).  Written as and/or of masked
  // entries: a select chain on r would be folded into a dynamically indexed
  // load, which forces the whole list out of registers into scratch.
  __device__ __forceinline__ u64 at(int r) const {
    u64 t = 0;
#pragma unroll
    for (int j = 0; j < KMAX; ++j) t |= key[j] & (0ull - (u64)(j == r));
    return t;
  }
};

}  // namespace mpl

namespace mpl {

// ------------------------------------------------------- cross-lane lists
// A group of G lanes (16 or 32, aligned within the wave) holds one sorted
// list: the lane of rank r (= lane % G) holds the r-th best key.

__device__ __forceinline__ u64 shfl_u64(u64 v, int src) {
  const uint32_t lo = __shfl((uint32_t)v, src);
  const uint32_t hi = __shfl((uint32_t)(v >> 32), src);
  return ((u64)hi << 32) | lo;
}

template <int G>
__device__ __forceinline__ u64 shfl_xor_u64(u64 v, int mask) {
  const uint32_t lo = __shfl_xor((uint32_t)v, mask, G);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), mask, G);
  return ((u64)hi << 32) | lo;
}

// acc <- best G of (acc, b), both sorted descending across the group; the
// float payload follows its key.  Bitonic split + G-wide bitonic merger.
template <int G>
__device__ __forceinline__ void group_merge(u64& acc, float& pay, u64 b, float bp, int r, int base) {
  const int src = base + (G - 1 - r);
  const u64 br = shfl_u64(b, src);
  const float bpr = __shfl(bp, src);
  const bool take = br > acc;
  acc = take ? br : acc;
  pay = take ? bpr : pay;
  constexpr int kStages = G == 32 ? 5 : 4;
#pragma unroll
  for (int st = 0; st < kStages; ++st) {
    const int s = (G / 2) >> st;
    const u64 o = shfl_xor_u64<G>(acc, s);
    const float op = __shfl_xor(pay, s, G);
    const bool other = (o > acc) != ((r & s) != 0);  // as in g16::merge
    acc = other ? o : acc;
    pay = other ? op : pay;
  }
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int s = G / 2; s >= 1; s >>= 1) v = fmaxf(v, __shfl_xor(v, s, G));
  return v;
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int s = G / 2; s >= 1; s >>= 1) v += __shfl_xor(v, s, G);
  return v;
}

}  // namespace mpl

namespace mpl {

// ------------------------------------------- 16-lane groups without LDS
// Lane exchanges inside aligned 16-lane rows on the VALU (DPP) or the
// swizzle network: xor 1 / 2 are quad permutes, xor 8 is a rotate by 8 of
// the row, xor 4 and the broadcasts are ds_swizzle bit patterns
// (lane' = ((lane & and) | or) ^ xor within 32 lanes).
namespace g16 {

template <int S>
__device__ __forceinline__ uint32_t xr(uint32_t v) {
  if constexpr (S == 1) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
  else if constexpr (S == 2) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
  else if constexpr (S == 4) return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (4 << 10) | 0x1F);
  else return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
}
// lane i of the row <- lane 15 - i
__device__ __forceinline__ uint32_t mirror(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false);
}
// every lane of the row <- lane I of the row
template <int I>
__device__ __forceinline__ uint32_t bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (I << 5) | 0x10);
}
// lane i <- lane i + 8 (lanes 8..15 receive 0)
__device__ __forceinline__ uint32_t shl8(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x108, 0xF, 0xF, true);
}

template <int S>
__device__ __forceinline__ u64 xr64(u64 v) {
  return ((u64)xr<S>((uint32_t)(v >> 32)) << 32) | xr<S>((uint32_t)v);
}
template <int S>
__device__ __forceinline__ float xrf(float v) {
  return __uint_as_float(xr<S>(__float_as_uint(v)));
}
template <int I>
__device__ __forceinline__ float bcastf(float v) {
  return __uint_as_float(bcast<I>(__float_as_uint(v)));
}

// acc <- best 16 of (acc, b), both sorted descending across the row (lane r
// holds rank r); payloads follow their keys.  Bitonic split against the
// mirrored b, then a 4-stage bitonic merger.  In a stage the lower lane of a
// pair keeps the larger key and the upper lane the smaller: the upper lane
// takes its partner's key unless that key is larger, so one compare serves
// both (equal keys are only the empty key 0, whose swap changes nothing that
// is output).
__device__ __forceinline__ void merge(u64& acc, float& pay, u64 b, float bp, int r) {
  const u64 br = ((u64)mirror((uint32_t)(b >> 32)) << 32) | mirror((uint32_t)b);
  const float bpr = __uint_as_float(mirror(__float_as_uint(bp)));
  const bool take = br > acc;
  acc = take ? br : acc;
  pay = take ? bpr : pay;
#define MPL_G16_STAGE(S)                                  \
  {                                                       \
    const u64 o = xr64<S>(acc);                           \
    const float op = xrf<S>(pay);                         \
    const bool upper = (r & S) != 0;                      \
    const bool other = (o > acc) != upper;                \
    acc = other ? o : acc;                                \
    pay = other ? op : pay;                               \
  }
  MPL_G16_STAGE(8)
  MPL_G16_STAGE(4)
  MPL_G16_STAGE(2)
  MPL_G16_STAGE(1)
#undef MPL_G16_STAGE
}

__device__ __forceinline__ float rmax(float v) {
  v = fmaxf(v, xrf<8>(v));
  v = fmaxf(v, xrf<4>(v));
  v = fmaxf(v, xrf<2>(v));
  return fmaxf(v, xrf<1>(v));
}
__device__ __forceinline__ float rsum(float v) {
  v += xrf<8>(v);
  v += xrf<4>(v);
  v += xrf<2>(v);
  return v + xrf<1>(v);
}

}  // namespace g16
}  // namespace mpl

namespace mpl {

// ------------------------------------------------ whole-wave sorted lists
// Exchanges with lane ^ S across the 64-lane wave, on the VALU only: DPP
// inside 16-lane rows for S < 16 (xor 4 as a shift left and a shift right
// on alternate banks of 4 lanes), v_permlane16_swap / v_permlane32_swap for
// 16 and 32.  Bitonic sorts and merges of u64 keys (the order of make_key).
namespace w64 {

template <int S>
__device__ __forceinline__ uint32_t xr(uint32_t v, int lane) {
  if constexpr (S == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
  } else if constexpr (S == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
  } else if constexpr (S == 4) {
    // banks 0 and 2 of a row (lanes 0-3, 8-11) take lane + 4 (row_shl:4),
    // banks 1 and 3 take lane - 4 (row_shr:4)
    const int t = __builtin_amdgcn_update_dpp(0, (int)v, 0x104, 0xF, 0x5, false);
    return (uint32_t)__builtin_amdgcn_update_dpp(t, (int)v, 0x114, 0xF, 0xA, false);
  } else if constexpr (S == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (S == 16) {
    // odd rows of the first operand swap with even rows of the second
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else {
    static_assert(S == 32, "lane xor of 1, 2, 4, 8, 16 or 32");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}

template <int S>
__device__ __forceinline__ u64 xr64(u64 v, int lane) {
  return ((u64)xr<S>((uint32_t)(v >> 32), lane) << 32) | xr<S>((uint32_t)v, lane);
}

// One compare-exchange stage with lane ^ S on N independent lists: the lane
// keeps the larger key when keep_max, else the smaller.
template <int S, int N>
__device__ __forceinline__ void stage(u64 (&v)[N], int lane, bool keep_max) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const u64 o = xr64<S>(v[i], lane);
    v[i] = ((o > v[i]) == keep_max) ? o : v[i];
  }
}

// Bitonic merge of stages S, S/2, ..., 1: each aligned group of 2S lanes
// holding a bitonic sequence ends sorted, descending where desc.
template <int S, int N>
__device__ __forceinline__ void merge_down(u64 (&v)[N], int lane, bool desc) {
  stage<S, N>(v, lane, ((lane & S) == 0) == desc);
  if constexpr (S > 1) merge_down<S / 2, N>(v, lane, desc);
}

// Sorts the wave's 64 keys of each list descending: lane r ends with rank r.
template <int N>
__device__ __forceinline__ void sort64_desc(u64 (&v)[N], int lane) {
  merge_down<1, N>(v, lane, (lane & 2) == 0);
  merge_down<2, N>(v, lane, (lane & 4) == 0);
  merge_down<4, N>(v, lane, (lane & 8) == 0);
  merge_down<8, N>(v, lane, (lane & 16) == 0);
  merge_down<16, N>(v, lane, (lane & 32) == 0);
  merge_down<32, N>(v, lane, true);
}

// Best 16 of four sorted 16-key lists, lane i holding entry i % 16 of list
// i / 16, lists 1 and 3 in reverse order (so lanes 0-31 and 32-63 are each
// a bitonic sequence).  Lanes 0-15 end with the best 16, descending.
template <int N>
__device__ __forceinline__ void best16_of4(u64 (&v)[N], int lane) {
#pragma unroll
  for (int i = 0; i < N; ++i) {  // lists 0+1 -> lanes 0-15, lists 2+3 -> lanes 32-47 (bitonic split)
    const u64 o = xr64<16>(v[i], lane);
    v[i] = o > v[i] ? o : v[i];
  }
  merge_down<8, N>(v, lane, (lane & 32) == 0);  // lanes 0-15 descending, 32-47 ascending
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const u64 o = xr64<32>(v[i], lane);
    v[i] = o > v[i] ? o : v[i];
  }
  merge_down<8, N>(v, lane, true);
}

}  // namespace w64
}  // namespace mpl
