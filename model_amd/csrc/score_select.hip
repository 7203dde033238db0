// Product-key selection: cosine scoring on MFMA fused with the exact stage-1
// top-k (memory.py:149-164), then stage-2 top-k over the k*k candidates and
// the routing softmax (memory.py:167-178).
//
// Stage 1 (score_topk_kernel).  A workgroup of two waves handles one
// codebook hc = h*2 + c and one split of its n sub-keys; each wave owns 32
// queries.  The queries are normalised in registers (or read normalised) and
// held as the MFMA B operand; each block of 32 keys is one chain of 32x32
// MFMAs (keys = A operand).  Key blocks reach the waves one of two ways,
// chosen per instantiation by register budget: each wave loads its own A
// operand two blocks ahead into registers (no LDS, no barriers; the faster
// path wherever the extra 32-64 VGPRs keep the occupancy), or the workgroup
// streams them through two LDS buffers by LDS DMA and shares them.
// Lanes l and l+32 share query l%32 and see alternate groups of 4 keys.  Two
// passes:
//   1. a bound pass over the first blocks of the split keeps, per register
//      position, the running maximum of the positive scores (-inf if none);
//      the k-th largest of a query's 32 maxima (the lane pair exchanges them
//      with v_permlane32_swap) is a score that at least k distinct keys
//      reach, so it bounds the k-th best from below;
//   2. a select pass over the whole split appends scores at or above the
//      lane's threshold to its column of an LDS buffer and, when any column
//      may overflow, sorts the buffered candidates in chunks of 8 and
//      bitonic-merges them into the lane's register list of the best k
//      (topk.h), raising the threshold to the k-th best so far.  At the end
//      the two lanes of a query merge their lists.
// Keys of equal score order by index, so the result is exactly lax.top_k's.
// The MFMAs of block j+1 are issued between the element steps of block j, so
// the matrix cores and the VALU overlap.  Scores never leave registers/LDS.
//
// Without routing noise the selection runs on the raw cosine: scores are
// cos*T(*q_len) with positive per-query factors, so the order is the same up
// to ties created by the rounding of that product (near-ties).
//
// Split plans.  Few tokens cannot fill the GPU with one workgroup per 64
// queries, so the key range of each codebook is split across workgroups and
// the per-split lists are merged (merge_splits_k16 reduces eight lists per
// 16-lane row at a time) before stage 2.
//
// Stage 2 (pair_kernel_k16 for k = 16, pair_kernel<G> otherwise).  A row of
// 16 lanes (k <= 16) or a group of 32 per (token, head) merges the lists of
// both codebooks, walks the k*k candidate grid as sorted row lists keyed by
// (select sum desc, flat index rank_a*k + rank_b asc) as memory.py:171, and
// finishes with the softmax of the clean slot scores (memory.py:178).  The
// k = 16 kernel exchanges values with DPP and ds_swizzle only.
#include <limits.h>

#include <algorithm>
#include <math.h>
#include <mutex>

#include "common.h"
#include "layout.h"
#include "mfma.h"
#include "topk.h"
#include "wsum.h"

namespace mpl {

#ifndef MPL_CAND
#define MPL_CAND 30
#endif
constexpr int kCand = MPL_CAND;  // per-lane candidate buffer (entries)
#ifndef MPL_NOISE_CAND
#define MPL_NOISE_CAND 22
#endif
constexpr int kNoiseCand = MPL_NOISE_CAND;  // the same with routing noise
#ifndef MPL_SCORE_THREADS
#define MPL_SCORE_THREADS 128
#endif
constexpr int kScoreThreads = MPL_SCORE_THREADS;  // waves per workgroup x 64
constexpr int kQueriesPerWave = 32;
constexpr int kQueriesPerGroup = kQueriesPerWave * (kScoreThreads / 64);
#ifndef MPL_MAX_SPLITS
#define MPL_MAX_SPLITS 64
#endif
constexpr int kMaxSplits = MPL_MAX_SPLITS;

struct ScoreParams {
  const void* q_hat;    // [M, HC, half]: normalised in the scoring type (mode 0) or raw fp32
  const float* q_len;   // [M, HC] or null (mode 0 input)
  float* out_qlen;      // [M, HC] or null (mode 2 output)
  int query_mode;       // MPL_Q_NORMALIZED / MPL_Q_RAW / MPL_Q_RAW_SCALED
  const uint4* packed;  // packed keys
  const float* gumbel;  // [M, HC, n] or null
  const float* T;           // device scalar: the clamped temperature
  const float* noise_coef;  // device scalar routing_noise * noise_scale (read with noise only)
  int noise_vec;  // gumbel rows 16-byte aligned (base aligned, n % 4 == 0)
  int64_t M;
  int HC, n, half, k, nblk, splits, blk_per_split;
  int pass1_blocks;  // blocks of each split scanned by the bound pass
  float* out_sel;    // [splits, HC, k, M] (null without noise: equals clean)
  float* out_clean;  // [splits, HC, k, M]
  int* out_idx;      // [splits, HC, k, M]
};

// Per-lane selection state of the stage-1 kernel.  Candidates are appended
// to the lane's column of two LDS arrays of [waves][entries][64] words
// (score, key index; with noise the score is the clean one, cand_entry);
// `off` is the byte offset of the lane's next free entry, the same in both.
// Entries of a column are 4*64 bytes apart.  The stores address the
// __shared__ arrays directly (array + byte offset, not a loop-carried
// pointer), so the compiler can tell them from the LDS-DMA writes of the key
// tiles (it does not wait for the in-flight DMA before an append) and folds
// each array's LDS address into the instruction's offset field: an append is
// one add and a ds_write2st64_b32 from one address register.
template <int KMAX, bool NOISE>
struct LaneSel {
  TopList<KMAX, NOISE> top;
  float thr;
  uint32_t off;
};
constexpr uint32_t kEntryBytes = 4 * kWave;

template <typename W>
__device__ __forceinline__ W& lds_at(W* arr, uint32_t byte_off) {
  return *(W*)((char*)arr + byte_off);
}

// KMAX-th largest key of the union of the lane pair's two sorted lists (the
// partner lane's arrives through v_permlane32_swap): the element-wise max of
// the own list and the partner's reversed list is the union's top KMAX as a
// bitonic sequence, so its minimum is the KMAX-th largest.  Both lanes of the
// pair get the same key; 0 when the union holds fewer than KMAX keys.
template <int KMAX, bool NOISE>
__device__ __forceinline__ u64 pair_kth_key(const TopList<KMAX, NOISE>& top, int par) {
  u64 m = ~0ull;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    float lo = __uint_as_float((uint32_t)top.key[j]), lo2 = lo;
    float hi = __uint_as_float((uint32_t)(top.key[j] >> 32)), hi2 = hi;
    half_swap(lo, lo2);
    half_swap(hi, hi2);
    const u64 other = ((u64)__float_as_uint(par ? hi : hi2) << 32) | __float_as_uint(par ? lo : lo2);
    const u64 own = top.key[KMAX - 1 - j];
    const u64 c = own > other ? own : other;
    m = c < m ? c : m;
  }
  return m;
}

// Key (and clean-score payload, with noise) of a buffered candidate at byte
// offset o.  Without noise the score array holds the select score.  With
// noise it holds the clean score, and the select score is formed again as
// the select pass formed it, fma(coef, gumbel[idx], clean), from the lane's
// noise row: the same bits, and one LDS array per candidate fewer.  Entries
// past the lane's count (!in) give the empty key.
template <bool NOISE>
__device__ __forceinline__ void cand_entry(const float* cs, const uint32_t* ci, const float* grow, float coef,
                                           uint32_t o, bool in, u64& key, float& pay) {
  const float v = lds_at(cs, o);
  const int id = in ? (int)lds_at(ci, o) : 0;
  if (NOISE) {
    const float g = grow[id];  // id < n: padded keys are never buffered
    key = in ? make_key(__builtin_fmaf(coef, g, v), id) : 0ull;
    pay = in ? v : 0.f;
  } else {
    key = in ? make_key(v, id) : 0ull;
    pay = 0.f;
  }
}

// Merges the lane's buffered candidates (entries lane0, lane0 + kEntryBytes,
// ... below st.off) into its list, empties the buffer and, with REFRESH,
// raises the threshold.  With k == KMAX the new threshold is the k-th best of
// both lanes of the query together (its k-th best so far), otherwise the
// lane's own k-th.  A key still to come that ties it loses on its larger
// index, so '>' against it keeps every key that can still enter.  Wave-uniform
// control flow.
//
// `empty` (wave-uniform): no flush has filled the list yet, so the first
// chunk, sorted, is the list's head as it stands (the rest of the list is
// empty keys) and needs no merge.
template <bool REFRESH, int KMAX, bool NOISE, int CAP>
__device__ __forceinline__ void flush_lane(LaneSel<KMAX, NOISE>& st, const float* cs, const uint32_t* ci,
                                           const float* grow, float coef, uint32_t lane0, bool valid, int k,
                                           float base_thr, int par, bool empty = false) {
  const int cnt = (int)((st.off - lane0) / kEntryBytes);
  // Rolled on purpose: this body is inlined at five sites of the block loop
  // and unrolled copies overflow the instruction cache.
#pragma unroll 1
  for (int c0 = 0; c0 < CAP; c0 += 8) {
    if (__ballot(c0 < cnt) == 0) break;
    u64 ch[8];
    float cp[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      cand_entry<NOISE>(cs, ci, grow, coef, lane0 + (uint32_t)(c0 + i) * kEntryBytes, c0 + i < cnt, ch[i], cp[i]);
    sort8<NOISE>(ch, cp);
    if (empty && c0 == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        st.top.key[i] = ch[i];
        if (NOISE) st.top.pay[NOISE ? i : 0] = cp[i];
      }
    } else {
      st.top.template merge<8>(ch, cp);
    }
  }
  st.off = lane0;
  if (REFRESH) {
    const u64 kk = k == KMAX ? pair_kth_key<KMAX, NOISE>(st.top, par) : st.top.at(k - 1);
    if (valid) st.thr = kk ? key_score(kk) : base_thr;
  }
}

// The final flush of a lane pair (lanes l and l + 32 share a query): the
// pair's buffered candidates are read as one sequence (the par-0 lane's
// column, cnt0 entries from base0, then the par-1 lane's from base1) and
// each lane merges an even share of it, entries [s, t), into its own list;
// the pair merge that follows combines the two lists.  A wave runs as many
// chunks of 8 as its fullest lane needs, so the split takes the wave's count
// from that of its fullest lane to that of its fullest pair, halved.
template <int KMAX, bool NOISE, int CAP>
__device__ __forceinline__ void flush_pair_range(LaneSel<KMAX, NOISE>& st, const float* cs, const uint32_t* ci,
                                                 const float* grow, float coef, int s, int t, int cnt0,
                                                 uint32_t base0, uint32_t base1, bool empty) {
  const int cnt = t - s;
#pragma unroll 1
  for (int c0 = 0; c0 < CAP; c0 += 8) {
    if (__ballot(c0 < cnt) == 0) break;
    u64 ch[8];
    float cp[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool in = c0 + i < cnt;
      const int e = s + c0 + i;
      const uint32_t o = !in ? base0 : e < cnt0 ? base0 + (uint32_t)e * kEntryBytes
                                                : base1 + (uint32_t)(e - cnt0) * kEntryBytes;
      cand_entry<NOISE>(cs, ci, grow, coef, o, in, ch[i], cp[i]);
    }
    sort8<NOISE>(ch, cp);
    if (empty && c0 == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        st.top.key[i] = ch[i];
        if (NOISE) st.top.pay[NOISE ? i : 0] = cp[i];
      }
    } else {
      st.top.template merge<8>(ch, cp);
    }
  }
}

// k-th largest (k <= 32) of the 32 floats a[0..15], b[0..15]: bitonic sort
// of the orderable bit patterns (max/min only), then a masked pick.
__device__ __forceinline__ float kth_of_32(const float* a, const float* b, int k) {
  uint32_t v[32];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    v[i] = orderable(a[i]);
    v[16 + i] = orderable(b[i]);
  }
#pragma unroll
  for (int size = 2; size <= 32; size <<= 1) {
#pragma unroll
    for (int stride = size / 2; stride >= 1; stride >>= 1) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;  // sort descending overall
          const uint32_t x = v[i], y = v[j];
          v[i] = desc ? max(x, y) : min(x, y);
          v[j] = desc ? min(x, y) : max(x, y);
        }
      }
    }
  }
  uint32_t t = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) t |= v[i] & (0u - (uint32_t)(i == k - 1));
  return from_orderable(t);
}

// k-th largest (k <= 16) of the 32 values of a lane pair, `own` here and the
// partner lane's in the other lane.  Each lane sorts its own 16 descending
// (bitonic, on orderable bits), the pair exchanges the sorted lists, and the
// element-wise max of the own list against the partner's reversed holds the
// top 16 of the 32 as a bitonic sequence, which a 4-stage merger sorts.
// Both lanes reach the same list.  About 330 VALU instructions against 770
// for kth_of_32 on the exchanged values.
__device__ __forceinline__ float kth_of_pair16(const float* own, int par, int k) {
  uint32_t v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = orderable(own[i]);
#pragma unroll
  for (int size = 2; size <= 16; size <<= 1) {
#pragma unroll
    for (int stride = size / 2; stride >= 1; stride >>= 1) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;
          const uint32_t x = v[i], y = v[j];
          v[i] = desc ? max(x, y) : min(x, y);
          v[j] = desc ? min(x, y) : max(x, y);
        }
      }
    }
  }
  uint32_t t[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float a = __uint_as_float(v[15 - i]), b = a;
    half_swap(a, b);  // the partner's entry 15 - i
    t[i] = max(v[i], __float_as_uint(par ? a : b));
  }
  if (k == 16) {  // the 16th largest of the 32 is the smallest of the top 16
    uint32_t m = t[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) m = min(m, t[i]);
    return from_orderable(m);
  }
#pragma unroll
  for (int stride = 8; stride >= 1; stride >>= 1) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if ((i & stride) == 0) {
        const uint32_t x = t[i], y = t[i + stride];
        t[i] = max(x, y);
        t[i + stride] = min(x, y);
      }
    }
  }
  uint32_t r = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) r |= t[i] & (0u - (uint32_t)(i == k - 1));
  return from_orderable(r);
}

// The wave's MFMA query operand: lane l holds query row my_q (= the wave's
// first query + l % 32), dims 16c + 8*(l/32) + [0,8) of chunk c (fp16; the
// fp32 tile's map for fp32), and ql, the row's length factor (1 without
// query_scale / q_len).  Rows out of range (!valid) are zeros.  With
// write_qlen, mode RAW_SCALED also stores ql to out_qlen.
template <typename T, int NCH>
__device__ __forceinline__ void query_operand(const ScoreParams& p, int hc, int64_t my_q, bool valid, int lane,
                                              bool write_qlen, typename Mfma<T>::Op (&qop)[NCH], float& ql) {
  const int par = lane >> 5;
  ql = 1.f;
  if (p.query_mode == MPL_Q_NORMALIZED) {
    const T* qrow = (const T*)p.q_hat + (valid ? (my_q * p.HC + hc) * (int64_t)p.half : 0);
#pragma unroll
    for (int c = 0; c < NCH; ++c) qop[c] = Mfma<T>::load_q(qrow, valid, p.half, c, lane);
    if (p.q_len != nullptr) ql = p.q_len[(valid ? my_q : 0) * p.HC + hc];
  } else {
    // Raw fp32 queries, normalised here (memory.py:30-31, 136-137): the
    // lane pair holds the row's 2*NCH*8 dims, so one half-swap completes
    // the sum of squares.
    const float* qrow = (const float*)p.q_hat + (valid ? (my_q * p.HC + hc) * (int64_t)p.half : 0);
    float x[NCH][Mfma<T>::kQElems];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) Mfma<T>::load_q_raw(qrow, valid, p.half, c, lane, x[c], ss);
    float a = ss, b = ss;
    half_swap(a, b);
    const float tot = ss + (par ? a : b) + 1e-6f;
    const float rn = 1.0f / sqrtf(tot);
#pragma unroll
    for (int c = 0; c < NCH; ++c) qop[c] = Mfma<T>::scale_q(x[c], rn);
    if (p.query_mode == MPL_Q_RAW_SCALED) {
      ql = sqrtf(tot) / sqrtf((float)p.half);
      if (p.out_qlen != nullptr && valid && write_qlen && par == 0) p.out_qlen[my_q * p.HC + hc] = ql;
    }
  }
}

// Short splits (SB = 4 or 8 blocks at most, no noise: the decode-sized
// plans): the workgroup copies all of the split's key blocks into LDS by LDS
// DMA at kernel start, each wave scores every block once from there, and
// both passes read the scores from the MFMA accumulators instead of
// reloading and re-scoring.  The key tiles lie in the candidate arrays,
// which the select pass takes over after a barrier; the arrays hold 64
// entries per lane, so SB = 4 needs no overflow check inside the pass and
// SB = 8 one per block from the fifth on.  SB = 0: the streaming passes.
constexpr int kShortCand = 64;
template <typename T, int HP>
constexpr bool short_fits(int sb) {
  return sb * KeyPack<T>::vectors_per_lane(HP) * kWave * 16 <= 2 * (kScoreThreads / kWave) * kShortCand * kWave * 4;
}

// Minimum waves per SIMD the compiler allocates registers for: the noisy
// fp16 selection with k <= 16 is held to two (its 38.5 KB of LDS per
// workgroup allows two per SIMD; without the bound it took 259 registers and
// ran at one).
template <typename T, bool NOISE, int KMAX>
constexpr int stage1_min_waves() {
  return (NOISE && KMAX == 16 && sizeof(T) == 2) ? 2 : 1;
}

template <typename T, int HP, bool NOISE, int KMAX, bool DIRECT, int SB>
__global__ __launch_bounds__(kScoreThreads, (stage1_min_waves<T, NOISE, KMAX>())) void score_topk_kernel(
    ScoreParams p) {
  constexpr int VPL = KeyPack<T>::vectors_per_lane(HP);  // 16-B vectors per lane per block
  constexpr int OPV = KeyPack<T>::kOpsPerVec;
  constexpr int NCH = VPL * OPV;                         // MFMA chunks per block
  constexpr int TILE = VPL * kWave;                      // uint4 per key block
  constexpr int WAVES = kScoreThreads / kWave;
  constexpr bool SHORT = SB > 0;
  typedef typename Mfma<T>::Op Op;
  static_assert(!SHORT || (!NOISE && short_fits<T, HP>(SB)), "short splits: no noise, key tiles fit the arrays");

  // with noise the buffer holds two arrays of 22 entries per lane (clean
  // score and index), so that with the key tiles a workgroup takes 38.5 KB of
  // LDS and two fit each SIMD
  constexpr int CAND = SHORT ? kShortCand : (NOISE ? kNoiseCand : kCand);
  __shared__ uint4 tile0[DIRECT || SHORT ? 1 : TILE], tile1[DIRECT || SHORT ? 1 : TILE];  // the LDS path's key tiles
  __shared__ float cscore[WAVES * CAND * kWave];
  __shared__ uint32_t cindex[WAVES * CAND * kWave];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int par = lane >> 5;  // key parity class of this lane
  const int hc = blockIdx.x % p.HC;
  const float Tv = *p.T;
  const float coef = NOISE ? *p.noise_coef : 0.f;
  const int split = (blockIdx.x / p.HC) % p.splits;
  const int64_t qb = blockIdx.x / (p.HC * p.splits);
  const int64_t q0 = qb * kQueriesPerGroup + wave * kQueriesPerWave;
  const int b_begin = split * p.blk_per_split;
  const int b_end = min(p.nblk, b_begin + p.blk_per_split);

  // Lanes l and l+32 own query q0 + l%32: the B operand holds that query, and
  // of each key block lane l scores keys 8*(r/4) + 4*par + r%4 (r < 16).
  const int64_t my_q = q0 + (lane & 31);
  const bool valid = my_q < p.M;

  const uint4* kbase_ptr = p.packed + (int64_t)hc * p.nblk * TILE;
  // The lane's VPL 16-byte vectors of key block blk (coalesced 1-KB loads).
  auto gload = [&](uint4* dst, int blk) __attribute__((always_inline)) {
    const uint4* src = kbase_ptr + (int64_t)blk * TILE + lane;
#pragma unroll
    for (int v = 0; v < VPL; ++v) dst[v] = src[v * kWave];
  };
  // Key blocks reach LDS by LDS DMA (global_load_lds: no registers, no LDS
  // store instructions).  Wave w copies the tile's 16-byte vectors w,
  // w+WAVES, ... (with fewer vectors than waves, several waves copy the same
  // bytes).
  constexpr int LPW = VPL >= WAVES ? VPL / WAVES : 1;
  static_assert(VPL < WAVES || VPL % WAVES == 0, "tile vectors must split over the waves");
  auto dma = [&](uint4* dst, int blk) __attribute__((always_inline)) {
    const uint4* src = kbase_ptr + (int64_t)blk * TILE;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int v = VPL >= WAVES ? wave + WAVES * i : wave % VPL;
      __builtin_amdgcn_global_load_lds((const void*)(src + v * kWave + lane), (lds_void*)(dst + v * kWave), 16, 0,
                                       0);
    }
  };
  // Short splits: tile j of the split in the candidate arrays (TPA tiles in
  // each), requested here for all blocks b_begin + j (clamped to the split,
  // so past its end a block repeats the last one) before the query, so that
  // keys and query arrive in one memory round trip.
  constexpr int TPA = (int)(sizeof(cscore) / (TILE * sizeof(uint4)));
  auto short_tile = [&](int j) __attribute__((always_inline)) {
    return j < TPA ? (uint4*)cscore + j * TILE : (uint4*)cindex + (j - TPA) * TILE;
  };
  if constexpr (SHORT) {
#pragma unroll
    for (int j = 0; j < SB; ++j) dma(short_tile(j), min(b_begin + j, b_end - 1));
  }

  Op qop[NCH];
  float ql;
  query_operand<T, NCH>(p, hc, my_q, valid, lane, split == 0, qop, ql);
  const float* grow = NOISE ? p.gumbel + ((valid ? my_q : 0) * p.HC + hc) * (int64_t)p.n : nullptr;
  const uint32_t lane0 = 4u * (uint32_t)(wave * CAND * kWave + lane);  // the lane's first buffer entry
  const uint32_t flush_at = lane0 + (uint32_t)(CAND - 8) * kEntryBytes;

  // The streaming LDS path: two key buffers, separate arrays used in a
  // compile-time alternation, so the compiler sees which buffer each LDS read
  // touches and does not drain the in-flight DMA of the other one before it.
  typedef float GVec __attribute__((ext_vector_type(NOISE ? 16 : 1)));
  // The lane's 16 noise values of block blk (keys 8*(r/4) + 4*par + r%4):
  // four 16-byte loads when the block is whole and the rows are 16-byte
  // aligned (noise_vec), else 16 clamped scalar loads.  The waits below count
  // kNoiseLoads outstanding noise loads; the scalar form only waits longer.
  constexpr int kNoiseLoads = NOISE ? 4 : 0;
  auto fetch_noise = [&](int blk) __attribute__((always_inline)) {
    GVec g;
    if (NOISE) {
      const int kb = blk * 32;
      if (p.noise_vec && kb + 32 <= p.n) {  // wave-uniform
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
          const float4 v = *(const float4*)(grow + kb + 8 * grp + 4 * par);
          g[NOISE ? 4 * grp + 0 : 0] = v.x;
          g[NOISE ? 4 * grp + 1 : 0] = v.y;
          g[NOISE ? 4 * grp + 2 : 0] = v.z;
          g[NOISE ? 4 * grp + 3 : 0] = v.w;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          g[NOISE ? r : 0] = grow[min(kb + 8 * (r >> 2) + 4 * par + (r & 3), p.n - 1)];
      }
    }
    return g;
  };
  // Register path (DIRECT): each wave loads its own A operand of block blk
  // into registers (gload) while the MFMAs of the block before it run; no
  // LDS tiles and no barriers.  Iteration j issues the loads of block j+2
  // into the registers of block j (whose MFMAs were issued in iteration
  // j-1), then waits for block j+1, issued one iteration earlier (loads
  // complete in order).
  auto sweep_direct = [&](int bb, int be, auto&& body) __attribute__((always_inline)) {
    const int nb = be - bb;
    if (nb <= 0) return;
    uint4 ua[VPL], ub[VPL];
    gload(ua, bb);
    gload(ub, min(bb + 1, be - 1));
    GVec gcur = fetch_noise(bb);
    wait_vmcnt_le<VPL + kNoiseLoads>();
    f32x16 x = f32x16{}, y;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
#pragma unroll
      for (int e = 0; e < OPV; ++e) x = Mfma<T>::mma(Mfma<T>::from_vec(ua[v], e), qop[v * OPV + e], x);
    }
    auto step = [&](int j, f32x16& c, f32x16& d, const uint4* ucur, uint4* unext) __attribute__((always_inline)) {
      gload(unext, min(bb + j + 2, be - 1));
      wait_vmcnt_le<VPL + kNoiseLoads>();
      d = f32x16{};
      auto issue = [&](int i) __attribute__((always_inline)) {
        d = Mfma<T>::mma(Mfma<T>::from_vec(ucur[i / OPV], i % OPV), qop[i], d);
      };
      const GVec gnext = fetch_noise(min(bb + j + 1, be - 1));
      body((bb + j) * 32, c, gcur, j < nb, issue);
      gcur = gnext;
    };
    for (int j = 0; j < nb; j += 2) {
      step(j, x, y, ub, ua);
      step(j + 1, y, x, ua, ub);
    }
  };
  // One sweep over key blocks [bb, be), software-pipelined: while the VALU
  // runs body() on block j, the MFMAs of block j+1 are already in flight.
  // Block j lives in buffer j % 2.  Iteration j: wait for this wave's DMA of
  // block j+1 (issued in iteration j-1; only the noise loads issued after it
  // may still be in flight: loads complete in order), join the barrier (so
  // every wave's DMA has landed and every wave has finished reading block j,
  // whose MFMAs were issued in iteration j-1), DMA block j+2 into block j's
  // buffer, then read block j+1 and run body() on block j with the next
  // block's MFMAs interleaved.  Past the end, DMAs copy clamped duplicates
  // and the one extra MFMA group scores one; nobody reads either.
  auto sweep_lds_on = [&](uint4* tile0, uint4* tile1, int bb, int be, auto&& body) __attribute__((always_inline)) {
    const int nb = be - bb;
    if (nb <= 0) return;
    dma(tile0, bb);
    dma(tile1, min(bb + 1, be - 1));
    GVec gcur = fetch_noise(bb);
    wait_vmcnt_le<LPW + kNoiseLoads>();
    asm volatile("s_barrier" ::: "memory");
    f32x16 x = f32x16{}, y;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const uint4 u = tile0[v * kWave + lane];
#pragma unroll
      for (int e = 0; e < OPV; ++e) x = Mfma<T>::mma(Mfma<T>::from_vec(u, e), qop[v * OPV + e], x);
    }
    // The MFMAs of the next block are issued unconditionally: a branch around
    // them would make the accumulator a phi, which the compiler resolves by
    // copying it right after the MFMAs, stalling on their results.  They are
    // handed to body() as issue(i), i < NCH, which body calls between its
    // element steps: a chain of dependent MFMAs issued back to back would
    // hold the wave's issue slot until each finishes.
    auto step = [&](int j, f32x16& c, f32x16& d, const uint4* rd, uint4* wr) __attribute__((always_inline)) {
      wait_vmcnt_le<kNoiseLoads>();
      // The wave's reads of `wr` (block j, read in iteration j - 1) must have
      // returned before any wave's DMA overwrites it: the compiler may sink
      // the MFMAs that consume them below this barrier, and with them the
      // wait for the reads.  A read still in flight when the DMA lands can
      // return a torn 16-byte vector (half of each key block), whose score
      // belongs to no key and can raise the bound pass's maxima above every
      // real score.
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      dma(wr, min(bb + j + 2, be - 1));
      uint4 u[VPL];
#pragma unroll
      for (int v = 0; v < VPL; ++v) u[v] = rd[v * kWave + lane];
      d = f32x16{};
      auto issue = [&](int i) __attribute__((always_inline)) {
        d = Mfma<T>::mma(Mfma<T>::from_vec(u[i / OPV], i % OPV), qop[i], d);
      };
      const GVec gnext = fetch_noise(min(bb + j + 1, be - 1));
      body((bb + j) * 32, c, gcur, j < nb, issue);
      gcur = gnext;
    };
    for (int j = 0; j < nb; j += 2) {
      step(j, x, y, tile1, tile0);
      step(j + 1, y, x, tile0, tile1);
    }
  };
  auto sweep_lds = [&](int bb, int be, auto&& body) __attribute__((always_inline)) {
    sweep_lds_on(tile0, tile1, bb, be, body);
  };

  f32x16 sacc[SHORT ? SB : 1];
  if constexpr (SHORT) {
    // every wave's DMA (and its query loads) landed: the scores of the
    // split's blocks (past the split's end a block repeats the last one,
    // which the passes skip or which leaves the maxima as they are)
    wait_vmcnt_le<0>();
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const uint4* tl = short_tile(j);
      f32x16 x = f32x16{};
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const uint4 u = tl[v * kWave + lane];
#pragma unroll
        for (int e = 0; e < OPV; ++e) x = Mfma<T>::mma(Mfma<T>::from_vec(u, e), qop[v * OPV + e], x);
      }
      sacc[SHORT ? j : 0] = x;
    }
    // both waves' tile reads are done before the select pass writes
    // candidates over the tiles
    __syncthreads();
  }
  auto sweep = [&](int bb, int be, auto&& body) __attribute__((always_inline)) {
    if constexpr (SHORT) {
      const GVec g{};
      auto no_issue = [](int) {};
#pragma unroll
      for (int j = 0; j < SB; ++j) body((bb + j) * 32, sacc[SHORT ? j : 0], g, j < be - bb, no_issue);
    } else if constexpr (DIRECT) {
      sweep_direct(bb, be, body);
    } else {
      sweep_lds(bb, be, body);
    }
  };

  // Selection values of the lane's 16 keys of a block (padded keys -inf);
  // with noise, cl holds the clean scores.
  // With noise, clean_at(c, r) is the clean score of element r; it is
  // recomputed where needed rather than kept in 16 more registers.
  auto clean_at = [&](const f32x16& c, int r) __attribute__((always_inline)) {
    float v = c[r] * Tv;
    return v * ql;  // ql == 1 without query_scale
  };
  auto lane_scores = [&](int kb, const f32x16& c, const GVec& g, float* sv) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      sv[r] = NOISE ? __builtin_fmaf(coef, g[NOISE ? r : 0], clean_at(c, r)) : c[r];
    if (kb + 32 > p.n) {  // wave-uniform: only the last block can hold padded keys
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (kb + 8 * (r >> 2) + 4 * par + (r & 3) >= p.n) sv[r] = -INFINITY;
    }
  };

  // Pass 1 over the first pass1_blocks blocks of the split: running maximum
  // per register position, taken as a signed-integer max of the float bit
  // patterns starting from -inf (one v_max_i32, no compare-select).  In that
  // order every positive score exceeds -inf and every negative one falls
  // below it, so each position ends with its largest positive score, or -inf
  // if it saw none.  Either way the 32 values of a lane pair (one query) are
  // scores of distinct keys or -inf, so their k-th largest is a lower bound
  // on that query's k-th best score; negative scores only loosen it.
  int ma[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) ma[r] = (int)0xff800000u;  // -inf
  const int p1_end = min(b_end, b_begin + p.pass1_blocks);
  // element r of 16 issues the next block's MFMA chunks [r*NCH/16, (r+1)*NCH/16)
  auto issue_for = [&](int r, auto&& issue) __attribute__((always_inline)) {
#pragma unroll
    for (int i = r * NCH / 16; i < (r + 1) * NCH / 16; ++i) issue(i);
  };
  auto bound_body = [&](int kb, const f32x16& c, const GVec& g, bool active, auto&& issue)
                        __attribute__((always_inline)) {
    float sv[16];
    const bool raw = !NOISE && kb + 32 <= p.n;  // wave-uniform
    if (!raw) lane_scores(kb, c, g, sv);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      issue_for(r, issue);
      const float v = raw ? c[r] : sv[r];
      // Past the end (!active) c holds a block of the split again (the last
      // one, or with SHORT a block pass 2 scans anyway), so its maxima are
      // still scores of this split's keys: no test of `active` is needed.
      ma[r] = max(ma[r], __float_as_int(v));
    }
    (void)active;
  };
  // The register path's bound pass streams each key block once per
  // workgroup: the waves' 8 KB loads from L2 held the pass at the L2's
  // delivery rate.  The block goes to LDS by DMA and both waves read it, in
  // two tiles laid over the candidate arrays (unused until the select pass,
  // which starts after every DMA has landed and both waves are past the
  // last tile read).  The select pass keeps register-loaded keys.
  constexpr bool LDS_BOUND = DIRECT && !SHORT && !NOISE && sizeof(cscore) >= TILE * sizeof(uint4) &&
                             sizeof(cindex) >= TILE * sizeof(uint4);
  if constexpr (LDS_BOUND) {
    sweep_lds_on((uint4*)cscore, (uint4*)cindex, b_begin, p1_end, bound_body);
    wait_vmcnt_le<0>();
    __syncthreads();
  } else {
    sweep(b_begin, p1_end, bound_body);
  }
  float fa[16];  // own maxima
#pragma unroll
  for (int r = 0; r < 16; ++r) fa[r] = __int_as_float(ma[r]);
  float bound;
  if constexpr (KMAX == 16) {
    bound = kth_of_pair16(fa, par, p.k);
  } else {
    float mb[16];  // the partner lane's maxima
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float a = fa[r], b = fa[r];
      half_swap(a, b);  // lane < 32: (own, partner); lane >= 32: (partner, own)
      mb[r] = par ? a : b;
    }
    bound = kth_of_32(fa, mb, p.k);
  }
  // Scores >= bound pass: strict '>' against the next float below it.  The
  // bound is never -0 (orderable maps it to +0), and below +0 the next float
  // that compares lower is -FLT_TRUE_MIN, two orderable steps down: one
  // step gives -0, which '>' does not separate from a score of exactly 0.
  const float base_thr =
      bound == -INFINITY ? -INFINITY : from_orderable(orderable(bound) - (bound == 0.f ? 2u : 1u));

  // Pass 2 over the whole split: only candidates above the threshold are
  // buffered and merged into the lane's sorted register list.
  LaneSel<KMAX, NOISE> st;
  st.top.init();
  st.thr = valid ? base_thr : INFINITY;
  st.off = lane0;
  bool flushed = false;  // wave-uniform: a flush inside the pass has filled the list
  // Every lane writes the element at its next free entry and keeps it only
  // when it is a candidate: no exec-mask changes per element (7 -> 4
  // instructions).  A kept-or-not write lands at or past the lane's last
  // candidate, which the flush does not read; the overflow checks leave room
  // for every element written before the next one.
  auto append8 = [&](int kb, const f32x16& c, const float* sv, bool active, int q, auto&& issue)
                     __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int r = 8 * q + e;
      issue_for(r, issue);
      const float x = sv[r];
      lds_at(cscore, st.off) = NOISE ? clean_at(c, r) : x;  // with noise the clean score (cand_entry)
      lds_at(cindex, st.off) = (uint32_t)(kb + 8 * (r >> 2) + 4 * par + (r & 3));
      st.off += (active && x > st.thr) ? kEntryBytes : 0u;
    }
  };
  if constexpr (SHORT) {
    // block j adds at most 16 entries to the 16 * j before it: from the
    // block that could overflow on, a check flushes above CAND - 16
    const uint32_t flush16 = lane0 + (uint32_t)(CAND - 16) * kEntryBytes;
    auto no_issue = [](int) {};
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int kb = (b_begin + j) * 32;
      const bool active = j < b_end - b_begin;
      if (16 * (j + 1) > CAND && active && __ballot(st.off > flush16) != 0) {
        flush_lane<true, KMAX, NOISE, CAND>(st, cscore, cindex, grow, coef, lane0, valid, p.k, base_thr, par);
        flushed = true;
      }
      float sv[16];
      const GVec g{};
      lane_scores(kb, sacc[SHORT ? j : 0], g, sv);
      append8(kb, sacc[SHORT ? j : 0], sv, active, 0, no_issue);
      append8(kb, sacc[SHORT ? j : 0], sv, active, 1, no_issue);
    }
  } else {
    sweep(b_begin, b_end, [&](int kb, const f32x16& c, const GVec& g, bool active, auto&& issue)
                              __attribute__((always_inline)) {
      float sv[16];
      lane_scores(kb, c, g, sv);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        // the flush check before each group of 8 leaves 8 free entries
        if (active && __ballot(st.off > flush_at) != 0) {
          flush_lane<true, KMAX, NOISE, CAND>(st, cscore, cindex, grow, coef, lane0, valid, p.k, base_thr, par);
          flushed = true;
        }
        append8(kb, c, sv, active, q, issue);
      }
    });
  }
  {
    const int cnt_own = (int)((st.off - lane0) / kEntryBytes);
    float ca = __int_as_float(cnt_own), cb = ca;
    half_swap(ca, cb);
    const int cnt_par = __float_as_int(par ? ca : cb);  // the partner lane's count
    const int cnt0 = par ? cnt_par : cnt_own;            // the par-0 lane's count
    const int tot = cnt_own + cnt_par, h = (tot + 1) >> 1;
    const uint32_t base0 = par ? lane0 - 4u * 32u : lane0;  // the par-0 lane's column
    flush_pair_range<KMAX, NOISE, CAND>(st, cscore, cindex, grow, coef, par ? h : 0, par ? tot : h, cnt0, base0,
                                  base0 + 4u * 32u, !flushed);
  }

  // Merge the two lanes' lists of the query: the partner's sorted list
  // arrives through v_permlane32_swap and is bitonic-merged (keys of the two
  // lanes are distinct: different key parities).
  {
    u64 other[KMAX];
    float opay[NOISE ? KMAX : 1];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      float lo = __uint_as_float((uint32_t)st.top.key[j]), lo2 = lo;
      float hi = __uint_as_float((uint32_t)(st.top.key[j] >> 32)), hi2 = hi;
      half_swap(lo, lo2);
      half_swap(hi, hi2);
      const float plo = par ? lo : lo2, phi = par ? hi : hi2;
      other[j] = ((u64)__float_as_uint(phi) << 32) | __float_as_uint(plo);
      if (NOISE) {
        float a = st.top.pay[NOISE ? j : 0], b = a;
        half_swap(a, b);
        opay[NOISE ? j : 0] = par ? a : b;
      }
    }
    st.top.template merge<KMAX>(other, opay);
  }

  if (valid && par == 0) {
    // Lists [split][M][hc][k]: lane l < 32 writes its query's k entries,
    // as 16-byte vectors when k == KMAX and the rows are 16-byte aligned.
    const int64_t o = (((int64_t)split * p.M + my_q) * p.HC + hc) * p.k;
    float cl[KMAX], se[KMAX];
    int id[KMAX];
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      const u64 kk = st.top.key[r];
      float clean, sel;
      if (NOISE) {
        clean = st.top.pay[NOISE ? r : 0];
        sel = key_score(kk);
      } else {
        clean = key_score(kk) * Tv;
        clean *= ql;  // ql == 1 without query_scale
        sel = clean;
      }
      if (kk == 0) clean = sel = -INFINITY;
      cl[r] = clean;
      se[r] = sel;
      id[r] = kk ? key_index(kk) : -1;
    }
    const bool vec = p.k == KMAX && ((uintptr_t)(p.out_clean + o) & 15) == 0 &&
                     ((uintptr_t)(p.out_idx + o) & 15) == 0 && (!NOISE || ((uintptr_t)(p.out_sel + o) & 15) == 0);
    if (vec) {
#pragma unroll
      for (int r = 0; r < KMAX; r += 4) {
        *(float4*)(p.out_clean + o + r) = make_float4(cl[r], cl[r + 1], cl[r + 2], cl[r + 3]);
        *(int4*)(p.out_idx + o + r) = make_int4(id[r], id[r + 1], id[r + 2], id[r + 3]);
        if (NOISE) *(float4*)(p.out_sel + o + r) = make_float4(se[r], se[r + 1], se[r + 2], se[r + 3]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < KMAX; ++r) {
        if (r < p.k) {
          if (NOISE) p.out_sel[o + r] = se[r];
          p.out_clean[o + r] = cl[r];
          p.out_idx[o + r] = id[r];
        }
      }
    }
  }
}

// ------------------------------------------------------- decode stage 1
// Decode-sized batches (M <= kDecodeMaxQ tokens, fp16 scoring, no routing
// noise): score_topk_decode<HP, MQ, WPG>.  A workgroup of WPG waves takes
// one codebook hc and 64*WPG consecutive keys, two key blocks per wave, for
// all M queries.  Scoring is score_topk_kernel's MFMA chain with the
// operands swapped (queries the A operand, keys the B operand): the tile's
// lane l holds key l % 32 and, in register q < 4, query q, and every score
// equals score_topk_kernel's bit for bit (the same products summed in the
// same order).  One v_permlane32_swap puts each query's 64 scores of the two
// blocks one per lane; a 64-lane bitonic sort leaves the wave's best 16 in
// lanes 0-15; the workgroup's lists meet in LDS and are reduced four at a
// time.  No bound pass and no candidate buffers: a decode wave has 64 keys
// per query, and the kernel's length is its memory round trip and the
// dependent exchange chain.
constexpr int kDecodeMaxQ = 4;
#ifndef MPL_DECODE_WAVES
#define MPL_DECODE_WAVES 4
#endif
constexpr int kDecodeWaves = MPL_DECODE_WAVES;  // waves per workgroup (4, 8 or 16)
static_assert(kDecodeWaves == 4 || kDecodeWaves == 8 || kDecodeWaves == 16, "decode workgroup of 4, 8 or 16 waves");

template <int HP, int MQ, int WPG>
__global__ __launch_bounds__(64 * WPG) void score_topk_decode(ScoreParams p) {
  typedef _Float16 T;
  constexpr int VPL = KeyPack<T>::vectors_per_lane(HP);
  constexpr int TILE = VPL * kWave;
  constexpr int NG = WPG / 4;  // workgroup lists after the first reduction
  typedef typename Mfma<T>::Op Op;
  __shared__ u64 wl[WPG][MQ][16];
  __shared__ u64 gl[NG > 1 ? NG : 1][MQ][16];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hc = blockIdx.x % p.HC;
  const int split = blockIdx.x / p.HC;
  const int b0 = split * p.blk_per_split + 2 * wave;  // the wave's blocks b0, b0 + 1
  const uint4* kb = p.packed + (int64_t)hc * p.nblk * TILE;
  // Both blocks' B operands (clamped past the last block; those keys are
  // dropped below), requested before the query: one memory round trip.
  uint4 kv[2][VPL];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint4* src = kb + (int64_t)min(b0 + j, p.nblk - 1) * TILE + lane;
#pragma unroll
    for (int v = 0; v < VPL; ++v) kv[j][v] = src[v * kWave];
  }
  __builtin_amdgcn_sched_barrier(0);
  const int64_t my_q = lane & 31;
  const bool valid = my_q < p.M;
  Op qop[VPL];
  float ql;
  query_operand<T, VPL>(p, hc, my_q, valid, lane, split == 0 && wave == 0, qop, ql);
  f32x16 x0 = f32x16{}, x1 = f32x16{};
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    x0 = Mfma<T>::mma(qop[v], Mfma<T>::from_vec(kv[0][v], 0), x0);
    x1 = Mfma<T>::mma(qop[v], Mfma<T>::from_vec(kv[1][v], 0), x1);
  }
  // Query q's scores: block b0 in lanes 0-31, block b0 + 1 in lanes 32-63.
  const int idx = (b0 + (lane >> 5)) * 32 + (lane & 31);
  u64 key[MQ];
#pragma unroll
  for (int q = 0; q < MQ; ++q) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x0[q]), __float_as_uint(x1[q]), false, false);
    const float s = __uint_as_float(r[0]);
    // padded keys and scores that are not above -inf (NaN included) are
    // never selected, as in score_topk_kernel
    key[q] = (idx < p.n && s > -INFINITY) ? make_key(s, idx) : 0ull;
  }
  w64::sort64_desc<MQ>(key, lane);
  if (lane < 16) {
#pragma unroll
    for (int q = 0; q < MQ; ++q) wl[wave][q][lane] = key[q];
  }
  __syncthreads();
  // lane i of a reducing wave loads entry i % 16 of list i / 16 of its group
  // of four, lists 1 and 3 reversed; lists past the end are empty
  auto load4 = [&](const u64 (*lists)[MQ][16], int first, int count) __attribute__((always_inline)) {
    const int t = lane >> 4, e = lane & 15;
    const int ent = (t & 1) ? 15 - e : e;
const int li = min(first + t, count - 1);
#pragma unroll
    for (int q = 0; q < MQ; ++q) {
      const u64 kk = lists[li][q][ent];
      key[q] = first + t < count ? kk : 0ull;
    }
    w64::best16_of4<MQ>(key, lane);
  };
  if constexpr (NG > 1) {
    if (wave < NG) {
      load4(wl, 4 * wave, WPG);
      if (lane < 16) {
#pragma unroll
        for (int q = 0; q < MQ; ++q) gl[wave][q][lane] = key[q];
      }
    }
    __syncthreads();
    if (wave != 0) return;
    load4(gl, 0, NG);
  } else {
    if (wave != 0) return;
    load4(wl, 0, WPG);
  }
  // Lists [split][M][hc][k]: lane r < k writes rank r of each query.
  const float Tv = *p.T;
  float qls[MQ];  // query q's length factor, from lane q
#pragma unroll
  for (int q = 0; q < MQ; ++q) qls[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ql), q));
  if (lane < p.k) {
#pragma unroll
    for (int q = 0; q < MQ; ++q) {
      if (q < p.M) {
        const float qlq = qls[q];
        const u64 kk = key[q];
        float clean = key_score(kk) * Tv;
        clean *= qlq;  // 1 without query_scale
        const int64_t o = (((int64_t)split * p.M + q) * p.HC + hc) * p.k + lane;
        p.out_clean[o] = kk ? clean : -INFINITY;
        p.out_idx[o] = kk ? key_index(kk) : -1;
      }
    }
  }
}

// ----------------------------------------------------------------- stage 2
// Stage-1 results arrive as "lists": sel / clean / idx arrays in the layout
// [split][M][hc][k] (sel absent without noise, where it equals clean).
// Ties each loaded list entry to a register at this point.  A value used
// only under a condition (an entry kept only when its id is valid) is
// otherwise loaded inside a branch with a wait of its own, after the other
// loads have returned: a second memory round trip.
template <int N>
__device__ __forceinline__ void pin_loaded(int (&id)[N], float (&sl)[N], float (&cc)[N]) {
#pragma unroll
  for (int t = 0; t < N; ++t) asm volatile("" ::"v"(id[t]), "v"(sl[t]), "v"(cc[t]));
}

struct PairParams {
  const float* sel;
  const float* clean;
  const int* idx;
  int64_t M;
  int H, n, k, S;
  int32_t* sub_idx;    // [M, HC, k] (written when S > 1)
  float* sub_scores;   // [M, HC, k] (written when S > 1)
  int32_t* flat_idx;   // [M, H, k]
  int32_t* slots;      // [M, H, k]
  float* weights;      // [M, H, k]
};

// A group of G lanes per (token, head).  Per codebook, the S split lists are
// combined with cross-lane bitonic merges (lane r ends with the rank-r
// entry).  The k*k candidates of memory.py:167-171 are then merged row by
// row as lists keyed (select sum, flat index rank_a*k + rank_b): row i holds
// k/(i+1) candidates that can still reach the top k, and the rows with a
// single such candidate (i >= k/2) form one more sorted list.  The softmax
// of memory.py:178 runs across the group.
template <int G>
__global__ __launch_bounds__(256) void pair_kernel(PairParams p) {
  const int lane = threadIdx.x & 63;
  const int r = lane % G;
  const int base = lane - r;
  const int64_t mh = ((int64_t)blockIdx.x * 256 + threadIdx.x) / G;
  const bool live = mh < p.M * p.H;  // dead groups still join the shuffles
  const int64_t m = live ? mh / p.H : 0;
  const int h = live ? (int)(mh % p.H) : 0;
  const int k = p.k;
  const int HC = 2 * p.H;
  const float* lsel = p.sel != nullptr ? p.sel : p.clean;

  u64 lk[2];
  float lc[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int hc = 2 * h + c;
    u64 acc = 0;
    float pay = 0.f;
    for (int s = 0; s < p.S; ++s) {
      const bool ok = live && r < k;
      const int64_t o = (((int64_t)s * p.M + m) * HC + hc) * k + (ok ? r : 0);  // clamped, unconditional
      const int id0 = p.idx[o];
      const float sl0 = lsel[o], cc0 = p.clean[o];
      const int id = ok ? id0 : -1;
      const u64 kk = id >= 0 ? make_key(sl0, id) : 0ull;
      const float cc = ok ? cc0 : 0.f;
      if (s == 0) {
        acc = kk;
        pay = cc;
      } else {
        group_merge<G>(acc, pay, kk, cc, r, base);
      }
    }
    lk[c] = acc;
    lc[c] = pay;
    if (p.S > 1 && live && r < k) {
      const int64_t so = (m * HC + hc) * k + r;
      p.sub_idx[so] = acc ? key_index(acc) : -1;
      p.sub_scores[so] = acc ? pay : -INFINITY;
    }
  }
  const bool a_ok = lk[0] != 0ull, b_ok = lk[1] != 0ull;
  const float a_sel = a_ok ? key_score(lk[0]) : -INFINITY;
  const float b_sel = b_ok ? key_score(lk[1]) : -INFINITY;
  const int a_id = a_ok ? key_index(lk[0]) : 0;
  const int b_id = b_ok ? key_index(lk[1]) : 0;
  const float a_cl = lc[0], b_cl = lc[1];

  // row 0: (0, j) at lane j
  const float a0 = __shfl(a_sel, base);
  const float a0c = __shfl(a_cl, base);
  const bool a0_ok = __shfl((int)a_ok, base) != 0;
  u64 acc = (r < k && a0_ok && b_ok) ? make_key(a0 + b_sel, r) : 0ull;
  float pay = a0c + b_cl;
  // rows 1 .. k/2-1: (i, j) for j < k/(i+1)
  for (int i = 1; i < k / 2; ++i) {
    const float ai = __shfl(a_sel, base + i);
    const float aic = __shfl(a_cl, base + i);
    const bool ai_ok = __shfl((int)a_ok, base + i) != 0;
    const u64 cand = (r < k / (i + 1) && ai_ok && b_ok) ? make_key(ai + b_sel, i * k + r) : 0ull;
    group_merge<G>(acc, pay, cand, aic + b_cl, r, base);
  }
  // rows max(1, k/2) .. k-1: only (i, 0) can reach the top k
  const int i0 = k / 2 > 1 ? k / 2 : 1;
  if (i0 < k) {
    const float b0 = __shfl(b_sel, base);
    const float b0c = __shfl(b_cl, base);
    const bool b0_ok = __shfl((int)b_ok, base) != 0;
    const int src = base + min(i0 + r, G - 1);
    const float ar = __shfl(a_sel, src);
    const float arc = __shfl(a_cl, src);
    const bool ar_ok = __shfl((int)a_ok, src) != 0;
    const u64 cand = (r < k - i0 && ar_ok && b0_ok) ? make_key(ar + b0, (i0 + r) * k) : 0ull;
    group_merge<G>(acc, pay, cand, arc + b0c, r, base);
  }

  // lane r < k holds the rank-r slot
  const int flat = acc ? key_index(acc) : 0;
  const int ra = min(flat / k, G - 1), rb = flat % k;
  int ia = __shfl(a_id, base + ra);
  int ib = __shfl(b_id, base + rb);
  // ids come from keys < n; the clamp only guards non-finite inputs
  ia = (ia >= 0 && ia < p.n) ? ia : 0;
  ib = (ib >= 0 && ib < p.n) ? ib : 0;
  const bool mine = r < k;
  const float sc = mine ? pay : -INFINITY;
  const float mx = group_max<G>(sc);
  const float e = mine ? expf(sc - mx) : 0.f;
  const float sum = group_sum<G>(e);
  if (live && mine) {
    const int64_t ob = mh * k + r;
    p.slots[ob] = ia * p.n + ib;
    p.flat_idx[ob] = flat;
    p.weights[ob] = e / sum;
  }
}

// pair_kernel for k == 16: the same algorithm on 16-lane rows with DPP /
// swizzle exchanges (no LDS traffic) and compile-time row broadcasts; split
// lists are loaded four at a time so their loads overlap.
// The pair stage of one (token, head) on a 16-lane row, from the two
// codebooks' final lists (lane r holds rank r of lk[c], clean score lc[c]):
// memory.py:167-175.  Writes slots, flat indices and routing weights of a
// live row.
// The lane's slot id (in [0, n*n)) and weight are also returned in slot_out
// and w_out, for a value read fused behind the pair stage.
__device__ __forceinline__ void pair_tail_k16(const PairParams& p, const u64 (&lk)[2], const float (&lc)[2],
                                              bool live, int64_t mh, int lane, int r, int& slot_out,
                                              float& w_out) {
  constexpr int K = 16;
  const bool a_ok = lk[0] != 0ull, b_ok = lk[1] != 0ull;
  const float a_sel = a_ok ? key_score(lk[0]) : -INFINITY;
  const float b_sel = b_ok ? key_score(lk[1]) : -INFINITY;
  const int a_id = a_ok ? key_index(lk[0]) : 0;
  const int b_id = b_ok ? key_index(lk[1]) : 0;
  const float a_cl = lc[0], b_cl = lc[1];
  const float aok = a_ok ? 1.f : 0.f;

  // The grid's candidate lists, each sorted descending across the row:
  // row i holds (i, j) for j < 16/(i+1) (rows 0..7), and list 8 the column
  // (i, 0) of rows 8..15 at lane i - 8.  They are merged as a tree, so the
  // merges of one level are independent and fill each other's exchange
  // latencies.
  u64 L[9];
  float P[9];
#define MPL_PAIR_ROW(I)                                                                                 \
  {                                                                                                     \
    const float ai = g16::bcastf<I>(a_sel), aic = g16::bcastf<I>(a_cl), aik = g16::bcastf<I>(aok);    \
    L[I] = (r < K / (I + 1) && aik != 0.f && b_ok) ? make_key(ai + b_sel, I * K + r) : 0ull;           \
    P[I] = aic + b_cl;                                                                                  \
  }
  MPL_PAIR_ROW(0) MPL_PAIR_ROW(1) MPL_PAIR_ROW(2) MPL_PAIR_ROW(3) MPL_PAIR_ROW(4) MPL_PAIR_ROW(5)
  MPL_PAIR_ROW(6) MPL_PAIR_ROW(7)
#undef MPL_PAIR_ROW
  {
    const float b0 = g16::bcastf<0>(b_sel), b0c = g16::bcastf<0>(b_cl);
    const bool b0_ok = b0 != -INFINITY;
    const float ar = __uint_as_float(g16::shl8(__float_as_uint(a_sel)));
    const float arc = __uint_as_float(g16::shl8(__float_as_uint(a_cl)));
    const float ark = __uint_as_float(g16::shl8(__float_as_uint(aok)));
    L[8] = (r < 8 && ark != 0.f && b0_ok) ? make_key(ar + b0, (8 + r) * K) : 0ull;
    P[8] = arc + b0c;
  }
#pragma unroll
  for (int i = 0; i < 8; i += 2) g16::merge(L[i], P[i], L[i + 1], P[i + 1], r);
  g16::merge(L[0], P[0], L[2], P[2], r);
  g16::merge(L[4], P[4], L[6], P[6], r);
  g16::merge(L[0], P[0], L[4], P[4], r);
  g16::merge(L[0], P[0], L[8], P[8], r);
  const u64 acc = L[0];
  const float pay = P[0];

  // lane r holds the rank-r slot
  const int flat = acc ? key_index(acc) : 0;
  const int base = lane - r;
  int ia = __shfl(a_id, base + flat / K);
  int ib = __shfl(b_id, base + flat % K);
  ia = (ia >= 0 && ia < p.n) ? ia : 0;  // ids come from keys < n; guards non-finite inputs
  ib = (ib >= 0 && ib < p.n) ? ib : 0;
  const float sc = acc ? pay : -INFINITY;
  const float mx = g16::rmax(sc);
  const float e = acc ? expf(sc - mx) : 0.f;
  const float sum = g16::rsum(e);
  slot_out = ia * p.n + ib;
  w_out = e / sum;
  if (live) {
    const int64_t ob = mh * K + r;
    p.slots[ob] = slot_out;
    p.flat_idx[ob] = flat;
    p.weights[ob] = w_out;
  }
}

// The two codebooks' final lists of row mh (lane r gets rank r of lk[c] and
// its clean score lc[c]): one split list loaded, or S lists merged.
__device__ __forceinline__ void pair_lists_k16(const PairParams& p, bool live, int64_t mh, int r, u64 (&lk)[2],
                                               float (&lc)[2]) {
  constexpr int K = 16;
  const int64_t m = live ? mh / p.H : 0;
  const int h = live ? (int)(mh % p.H) : 0;
  const int HC = 2 * p.H;
  const float* lsel = p.sel != nullptr ? p.sel : p.clean;

  // Dead rows read row 0 and enter as empty keys, whose payload is never
  // output.  Both codebooks' entries of a batch of lists are requested before
  // the first merge: one memory round trip per batch, and with one list no
  // merge at all.
  int64_t o0[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) o0[c] = ((int64_t)m * HC + 2 * h + c) * K + r;
  if (p.S == 1) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      int id[1] = {p.idx[o0[c]]};
      float sl[1] = {lsel[o0[c]]}, cc[1] = {p.clean[o0[c]]};
      pin_loaded(id, sl, cc);
      lc[c] = cc[0];
      lk[c] = (live && id[0] >= 0) ? make_key(sl[0], id[0]) : 0ull;
    }
  } else {
    constexpr int B = 8;
    const int64_t sstride = p.M * HC * K;
    for (int s0 = 0; s0 < p.S; s0 += B) {
      int id[2][B];
      float sl[2][B], cc[2][B];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int t = 0; t < B; ++t) {
          const int64_t o = (int64_t)min(s0 + t, p.S - 1) * sstride + o0[c];  // clamped, unconditional
          id[c][t] = p.idx[o];
          sl[c][t] = lsel[o];
          cc[c][t] = p.clean[o];
        }
#pragma unroll
      for (int c = 0; c < 2; ++c) pin_loaded(id[c], sl[c], cc[c]);
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int t = 0; t < B; ++t) {
          if (s0 + t < p.S) {  // uniform
            const u64 kk = (live && id[c][t] >= 0) ? make_key(sl[c][t], id[c][t]) : 0ull;
            if (s0 + t == 0) {
              lk[c] = kk;
              lc[c] = cc[c][t];
            } else {
              g16::merge(lk[c], lc[c], kk, cc[c][t], r);
            }
          }
        }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c)
      if (live) {
        p.sub_idx[o0[c]] = lk[c] ? key_index(lk[c]) : -1;
        p.sub_scores[o0[c]] = lk[c] ? lc[c] : -INFINITY;
      }
  }
}

__global__ __launch_bounds__(256) void pair_kernel_k16(PairParams p) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int64_t mh = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;
  const bool live = mh < p.M * p.H;  // dead rows still join the exchanges
  u64 lk[2];
  float lc[2];
  pair_lists_k16(p, live, mh, r, lk, lc);
  int slot;
  float w;
  pair_tail_k16(p, lk, lc, live, mh, lane, r, slot, w);
}

// The value read of a fused lookup (memory.py:179-193): values [n*n, VR*16
// bytes] of type V, read(s) = s or (s + N/2 + 1) % N (memory.py:179).
struct ReadParams {
  const void* values;
  int shuffle;
  float* out;  // [M, d] fp32
};

// Stage 2 and the value read in one kernel, for H = 4 and k = 16: the wave's
// four 16-lane rows are the four heads of one token, so after the pair stage
// lane h*16 + r holds that token's row h*k + r (slot and weight), exactly the
// lane layout the weighted row sum takes.  While some waves run the pair
// merges (VALU-bound), others have their row loads in flight.
template <typename V, int VR, bool NT>
__global__ __launch_bounds__(256) void pair_read_k16(PairParams p, ReadParams rp) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int64_t mh = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;
  const bool live = mh < p.M * 4;  // H = 4: a wave is live or dead as a whole
  u64 lk[2];
  float lc[2];
  pair_lists_k16(p, live, mh, r, lk, lc);
  int slot;
  float w;
  pair_tail_k16(p, lk, lc, live, mh, lane, r, slot, w);
  if (!live) return;
  const int64_t m = mh >> 2;
  const int64_t N = (int64_t)p.n * p.n;
  if (rp.shuffle) slot = (int)(((int64_t)slot + N / 2 + 1) % N);
  Wsum<V, VR, 16, NT> acc;
  acc.add_chunk((const uint4*)rp.values, slot, w, 64, lane);
  acc.store(rp.out + m * (int64_t)(VR * Vec16<V>::kElems), lane);
}

// Split lists are reduced eight at a time before stage 2 (k == 16 only).
constexpr int kMergeChunk = 8;

// Split-list reduction for k == 16: 16-lane row (s2, m, hc) merges lists
// s2*8 .. s2*8+7 of (m, hc) (loaded four at a time) into list s2.
struct MergeParams {
  const float* sel;  // null without noise (equals clean)
  const float* clean;
  const int* idx;
  int64_t rows;  // M * HC
  int S, S2;
  float* out_sel;
  float* out_clean;
  int* out_idx;
};

__global__ __launch_bounds__(256) void merge_splits_k16(MergeParams p) {
  constexpr int K = 16;
  const int r = threadIdx.x & 15;
  const int64_t g = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;
  const bool live = g < p.rows * p.S2;  // dead rows still join the exchanges
  const int64_t row = live ? g % p.rows : 0;
  const int s2 = live ? (int)(g / p.rows) : 0;
  const float* lsel = p.sel != nullptr ? p.sel : p.clean;
  const int64_t sstride = p.rows * K;
  // All lists of the chunk are requested before the first merge (one memory
  // round trip).  Lists past p.S read the last list again and enter as empty
  // keys; an empty key's payload is never output, so it is passed as loaded.
  int id[kMergeChunk];
  float sl[kMergeChunk], cc[kMergeChunk];
#pragma unroll
  for (int t = 0; t < kMergeChunk; ++t) {
    const int s = min(s2 * kMergeChunk + t, p.S - 1);  // clamped, unconditional
    const int64_t o = (int64_t)s * sstride + row * K + r;
    id[t] = p.idx[o];
    sl[t] = lsel[o];
    cc[t] = p.clean[o];
  }
  pin_loaded(id, sl, cc);
  u64 acc = 0;
  float pay = 0.f;
#pragma unroll
  for (int t = 0; t < kMergeChunk; ++t) {
    const bool in = s2 * kMergeChunk + t < p.S;  // uniform per row
    const u64 kk = (in && id[t] >= 0) ? make_key(sl[t], id[t]) : 0ull;
    if (t == 0) {
      acc = kk;
      pay = cc[t];
    } else {
      g16::merge(acc, pay, kk, cc[t], r);
    }
  }
  if (live) {
    const int64_t o = ((int64_t)s2 * p.rows + row) * K + r;
    p.out_idx[o] = acc ? key_index(acc) : -1;
    p.out_clean[o] = acc ? pay : -INFINITY;
    if (p.out_sel != nullptr) p.out_sel[o] = acc ? key_score(acc) : -INFINITY;
  }
}

// Stage 2 of a select with 8 < S <= 64 split lists (k == 16, the decode
// plans) in one launch instead of a merge_splits_k16 level plus the pair
// kernel: one workgroup per (token, head).  Row g of its 16 rows of 16 lanes
// merges lists 8*(g%8) .. 8*(g%8)+7 of codebook g/8 (lists past S enter as
// empty keys); the row lists meet in LDS, rows 0 and 8 merge their
// codebook's eight (the codebook's top-k, written to sub_idx / sub_scores),
// and row 0 runs the pair stage.
constexpr int kWideMaxSplits = kMergeChunk * kMergeChunk;

__global__ __launch_bounds__(256) void pair_wide_k16(PairParams p) {
  constexpr int K = 16;
  __shared__ u64 skey[16][K];
  __shared__ float spay[16][K];
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = threadIdx.x >> 4;
  const int c = g >> 3, chunk = g & 7;
  const int64_t mh = blockIdx.x;  // the grid is exactly M * H workgroups
  const int64_t m = mh / p.H;
  const int h = (int)(mh % p.H);
  const int HC = 2 * p.H;
  const float* lsel = p.sel != nullptr ? p.sel : p.clean;
  const int64_t o0 = ((int64_t)m * HC + 2 * h + c) * K + r;
  const int64_t sstride = p.M * HC * K;
  int id[kMergeChunk];
  float sl[kMergeChunk], cc[kMergeChunk];
#pragma unroll
  for (int t = 0; t < kMergeChunk; ++t) {
    const int64_t o = (int64_t)min(chunk * kMergeChunk + t, p.S - 1) * sstride + o0;  // clamped, unconditional
    id[t] = p.idx[o];
    sl[t] = lsel[o];
    cc[t] = p.clean[o];
  }
  pin_loaded(id, sl, cc);
  u64 acc = 0;
  float pay = 0.f;
#pragma unroll
  for (int t = 0; t < kMergeChunk; ++t) {
    const bool in = chunk * kMergeChunk + t < p.S;  // uniform per row
    const u64 kk = (in && id[t] >= 0) ? make_key(sl[t], id[t]) : 0ull;
    if (t == 0) {
      acc = kk;
      pay = cc[t];
    } else {
      g16::merge(acc, pay, kk, cc[t], r);
    }
  }
  skey[g][r] = acc;
  spay[g][r] = pay;
  __syncthreads();
  if (chunk == 0) {  // rows 0 and 8 read rows 1..7 and 9..15 and rewrite only their own entries
#pragma unroll
    for (int t = 1; t < kMergeChunk; ++t) g16::merge(acc, pay, skey[g + t][r], spay[g + t][r], r);
    p.sub_idx[o0] = acc ? key_index(acc) : -1;
    p.sub_scores[o0] = acc ? pay : -INFINITY;
    skey[g][r] = acc;
    spay[g][r] = pay;
  }
  __syncthreads();
  if (g == 0) {
    const u64 lk[2] = {skey[0][r], skey[8][r]};
    const float lc[2] = {spay[0][r], spay[8][r]};
    int slot;
    float w;
    pair_tail_k16(p, lk, lc, true, mh, lane, r, slot, w);
  }
}

// pair_wide_k16 fused with the value read, for H = 4: one workgroup per
// token, quarter h (256 threads) merges head h's split lists and runs its
// pair stage exactly as pair_wide_k16 does; the four heads' 16 (slot,
// weight) rows meet in LDS and wave 0 reads the token's 64 rows with the
// weighted row sum of wsum.h (the lane layout gather_wsum_kernel uses, so
// `out` equals the two-launch path bit for bit).  Decode-sized batches: one
// launch and one dependent memory round trip fewer than pair_wide_k16 +
// gather_wsum_kernel.
template <typename V, int VR, bool NT>
__global__ __launch_bounds__(1024) void pair_wide_read_k16(PairParams p, ReadParams rp) {
  constexpr int K = 16;
  __shared__ u64 skey[4][16][K];
  __shared__ float spay[4][16][K];
  __shared__ int srow_slot[4 * K];
  __shared__ float srow_w[4 * K];
  const int h = threadIdx.x >> 8;  // head of this quarter (H = 4)
  const int t = threadIdx.x & 255;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = t >> 4;
  const int c = g >> 3, chunk = g & 7;
  const int64_t m = blockIdx.x;  // the grid is exactly M workgroups
  const int64_t mh = m * 4 + h;
  const int HC = 8;
  const float* lsel = p.sel != nullptr ? p.sel : p.clean;
  const int64_t o0 = ((int64_t)m * HC + 2 * h + c) * K + r;
  const int64_t sstride = p.M * HC * K;
  int id[kMergeChunk];
  float sl[kMergeChunk], cc[kMergeChunk];
#pragma unroll
  for (int i = 0; i < kMergeChunk; ++i) {
    const int64_t o = (int64_t)min(chunk * kMergeChunk + i, p.S - 1) * sstride + o0;  // clamped, unconditional
    id[i] = p.idx[o];
    sl[i] = lsel[o];
    cc[i] = p.clean[o];
  }
  pin_loaded(id, sl, cc);
  u64 acc = 0;
  float pay = 0.f;
#pragma unroll
  for (int i = 0; i < kMergeChunk; ++i) {
    const bool in = chunk * kMergeChunk + i < p.S;  // uniform per row
    const u64 kk = (in && id[i] >= 0) ? make_key(sl[i], id[i]) : 0ull;
    if (i == 0) {
      acc = kk;
      pay = cc[i];
    } else {
      g16::merge(acc, pay, kk, cc[i], r);
    }
  }
  skey[h][g][r] = acc;
  spay[h][g][r] = pay;
  __syncthreads();
  if (chunk == 0) {  // rows 0 and 8 of each quarter read rows 1..7 and 9..15 and rewrite only their own
#pragma unroll
    for (int i = 1; i < kMergeChunk; ++i) g16::merge(acc, pay, skey[h][g + i][r], spay[h][g + i][r], r);
    p.sub_idx[o0] = acc ? key_index(acc) : -1;
    p.sub_scores[o0] = acc ? pay : -INFINITY;
    skey[h][g][r] = acc;
    spay[h][g][r] = pay;
  }
  __syncthreads();
  if (g == 0) {  // lanes 0-15 of the quarter's first wave
    const u64 lk[2] = {skey[h][0][r], skey[h][8][r]};
    const float lc[2] = {spay[h][0][r], spay[h][8][r]};
    int slot;
    float w;
    pair_tail_k16(p, lk, lc, true, mh, lane, r, slot, w);
    srow_slot[h * K + r] = slot;
    srow_w[h * K + r] = w;
  }
  __syncthreads();
  if (threadIdx.x < kWave) {  // wave 0: lane i holds row i = h * 16 + r of the token
    const int64_t N = (int64_t)p.n * p.n;
    int slot = srow_slot[lane];
    if (rp.shuffle) slot = (int)(((int64_t)slot + N / 2 + 1) % N);
    Wsum<V, VR, 16, NT> sum;
    sum.add_chunk((const uint4*)rp.values, slot, srow_w[lane], 64, lane);
    sum.store(rp.out + m * (int64_t)(VR * Vec16<V>::kElems), lane);
  }
}

// Stage 2 + value read for decode plans: 8 < S <= kDecodeMaxSplits split
// lists, no noise (the lists' select score is the clean score, so a list
// entry is its key alone), H = 4, k = 16, one row group per lane (VR <= 64).
// One workgroup of 16 waves per token, every exchange on the VALU.  SC (32
// or 64) is the split capacity:
//   1. wave w takes SC/2 lists of one codebook of head w % 4 (groups of four,
//      w64::best16_of4): the SC lists of a codebook become SC/4, in LDS;
//   2. wave h (< 4) reduces its head's lists to one per codebook (the
//      codebooks' top-k, written to sub_idx / sub_scores), then runs the
//      pair stage: of the k*k pairs (i, j) only the 50 with
//      (i+1)(j+1) <= 16 can be among the best 16 (every pair (i', j') with
//      i' <= i, j' <= j ranks before (i, j)), one per lane, and a 64-lane
//      sort orders them by (select sum desc, flat index i*k + j asc), as
//      memory.py:171-175; the softmax of the clean sums (memory.py:178) is
//      pair_tail_k16's, row exchanges included, so weights match it bit
//      for bit;
//   3. each head's wave issues the loads of its 16 rows as soon as its
//      weights are known (one memory round trip per head, the four heads
//      overlapping) and puts them in LDS; wave 0 then adds the token's row
//      groups in add_chunk's order, so `out` equals the two-launch path.
constexpr int kDecodeMaxSplits = 64;

template <typename V, int VR, bool NT, int SC>
__global__ __launch_bounds__(1024) void pair_decode_read_k16(PairParams p, ReadParams rp) {
  constexpr int K = 16;
  typedef Wsum<V, VR, 16, NT> Sum;
  static_assert(Sum::VPL == 1, "one vector per lane per row group");
  static_assert(SC == 32 || SC == 64, "split capacity 32 or 64");
  constexpr int RPI = Sum::RPI, LPR = Sum::LPR;
  constexpr int GROUPS = 64 / RPI;  // row groups of the token's 64 rows
  constexpr int HG = GROUPS / 4;     // row groups of one head
  constexpr int G1 = SC / 8;         // groups of four lists per wave in step 1
  constexpr int GPC = G1 / 2;        // groups per codebook in step 2
  __shared__ u64 l1[4][2][2 * G1][K];  // [head][codebook][list][rank] after step 1
  __shared__ u64 l2[4][G1][K];         // [head][list] within step 2
  __shared__ u64 pab[4][2][K];         // [head][codebook] final lists
  __shared__ float srow_w[4 * K];
  __shared__ uint4 rows[GROUPS][kWave];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t m = blockIdx.x;  // the grid is exactly M workgroups
  const int HC = 8;
  const int64_t sstride = p.M * HC * K;
  const int t = lane >> 4, e = lane & 15;
  const int ent = (t & 1) ? 15 - e : e;  // list t of a group of four, odd ones reversed
  {
    // step 1: wave w, head h = w % 4, codebook cb = (w / 4) >> 1 of the
    // head, lists (SC/2) * ((w / 4) & 1) + 4 * grp + t; past S empty
    const int h = wave & 3, sub = wave >> 2, cb = sub >> 1;
    const int c = 2 * h + cb;
    int id[G1];
    float cl[G1];
#pragma unroll
    for (int grp = 0; grp < G1; ++grp) {
      const int s = (SC / 2) * (sub & 1) + 4 * grp + t;
      const int64_t o = (int64_t)min(s, p.S - 1) * sstride + (m * HC + c) * K + ent;  // clamped, unconditional
      id[grp] = p.idx[o];
      cl[grp] = p.clean[o];
    }
    u64 key[G1];
#pragma unroll
    for (int grp = 0; grp < G1; ++grp) {
      const int s = (SC / 2) * (sub & 1) + 4 * grp + t;
      key[grp] = (s < p.S && id[grp] >= 0) ? make_key(cl[grp], id[grp]) : 0ull;
    }
    w64::best16_of4<G1>(key, lane);
    if (lane < K) {
#pragma unroll
      for (int grp = 0; grp < G1; ++grp) l1[h][cb][G1 * (sub & 1) + grp][lane] = key[grp];
    }
  }
  __syncthreads();
  if (wave < 4) {
    const int h = wave;
    // step 2a: group g holds lists 4 * (g % GPC) + t of codebook g / GPC
    u64 key[G1];
#pragma unroll
    for (int g = 0; g < G1; ++g) key[g] = l1[h][g / GPC][4 * (g % GPC) + t][ent];
    w64::best16_of4<G1>(key, lane);
    if (lane < K) {
#pragma unroll
      for (int g = 0; g < G1; ++g) l2[h][g][lane] = key[g];
    }
    // step 2b: each codebook's GPC lists to one, codebook 0 in lanes 0-15
    // and codebook 1 in lanes 32-47
    u64 fk;
    if constexpr (GPC == 2) {
      // lanes 0-31 hold codebook 0's two lists, lanes 32-63 codebook 1's
      // (second of each reversed): one bitonic split and a 16-lane merger
      u64 v[1] = {l2[h][t][ent]};
      const u64 o = w64::xr64<16>(v[0], lane);
      v[0] = o > v[0] ? o : v[0];
      w64::merge_down<8, 1>(v, lane, true);
      fk = v[0];
    } else {
      u64 v[2] = {l2[h][t][ent], l2[h][4 + t][ent]};  // a group of four per codebook
      w64::best16_of4<2>(v, lane);
      const u64 b = w64::xr64<32>(v[1], lane);  // codebook 1's list to lanes 32-47
      fk = (lane & 32) ? b : v[0];
    }
    if ((lane & 16) == 0) {  // lanes 0-15: codebook 2h, lanes 32-47: 2h + 1
      const int cb = lane >> 5;
      const int64_t o0 = (m * HC + 2 * h + cb) * K + e;
      p.sub_idx[o0] = fk ? key_index(fk) : -1;
      p.sub_scores[o0] = fk ? key_score(fk) : -INFINITY;
      pab[h][cb][e] = fk;
    }
    // the pair stage: lane l < 50 takes candidate (i, j), the l-th pair with
    // (i+1)(j+1) <= 16 in row-major order
    int pi = 0, pj = lane;
    bool found = false;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const int cnt = K / (i + 1);
      const bool here = !found && pj < cnt;
      pi = here ? i : pi;
      pj = (!found && !here) ? pj - cnt : pj;
      found = found || here;
    }
    const u64 ka = pab[h][0][pi], kb = pab[h][1][found ? pj : 0];
    const bool ok = found && ka != 0ull && kb != 0ull;
    u64 pk[1] = {ok ? make_key(key_score(ka) + key_score(kb), pi * K + pj) : 0ull};
    w64::sort64_desc<1>(pk, lane);
    const u64 acc = pk[0];
    // lane r < 16 holds the rank-r pair (as pair_tail_k16)
    const int flat = acc ? key_index(acc) : 0;
    const u64 wa = pab[h][0][flat / K], wb = pab[h][1][flat % K];
    int ia = wa ? key_index(wa) : 0;
    int ib = wb ? key_index(wb) : 0;
    ia = (ia >= 0 && ia < p.n) ? ia : 0;  // ids come from keys < n; guards non-finite inputs
    ib = (ib >= 0 && ib < p.n) ? ib : 0;
    const float pay = (wa ? key_score(wa) : -INFINITY) + (wb ? key_score(wb) : -INFINITY);
    const float sc = acc ? pay : -INFINITY;
    const float mx = g16::rmax(sc);
    const float ex = acc ? expf(sc - mx) : 0.f;
    const float sum = g16::rsum(ex);
    const int slot = ia * p.n + ib;
    const float w = ex / sum;
    const int64_t mh = m * 4 + h;
    if (lane < K) {
      const int64_t ob = mh * K + lane;
      p.slots[ob] = slot;
      p.flat_idx[ob] = flat;
      p.weights[ob] = w;
      srow_w[h * K + lane] = w;
    }
    // step 3: the head's rows (row groups HG * h ..), loaded at once
    const int64_t N = (int64_t)p.n * p.n;
    const int rs = rp.shuffle ? (int)(((int64_t)slot + N / 2 + 1) % N) : slot;
    uint4 buf[HG];
#pragma unroll
    for (int g = 0; g < HG; ++g) {
      const int rr = g * RPI + lane / LPR;  // row of the head, 0..15
      const int sr = __shfl(rs, rr);
      const uint4* src = (const uint4*)rp.values + (int64_t)sr * VR + lane % LPR;
      buf[g] = NT ? load_nt(src) : *src;
    }
#pragma unroll
    for (int g = 0; g < HG; ++g) rows[h * HG + g][lane] = buf[g];
  }
  __syncthreads();
  if (wave == 0) {
    Sum acc;
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) acc.add_vec(rows[g][lane], srow_w[g * RPI + lane / LPR]);
    acc.store(rp.out + m * (int64_t)(VR * Vec16<V>::kElems), lane);
  }
}

// ---------------------------------------------------------------- host side
struct Plan {
  int splits, blk_per_split, nblk, kmax, pass1_blocks;
  int64_t qblocks;
};

// Workgroups a launch should reach before the key range is split (two waves
// each: two waves per SIMD of the 256 CUs, so that one wave's selection work
// overlaps the other's MFMAs).
#ifndef MPL_SCORE_TARGET_WGS
#define MPL_SCORE_TARGET_WGS 1024
#endif
// The bound pass scans min(blocks, max(MIN, blocks / DIV)) blocks of a split.
#ifndef MPL_PASS1_MIN
#define MPL_PASS1_MIN 16
#endif
#ifndef MPL_PASS1_DIV
#define MPL_PASS1_DIV 8
#endif

static Plan make_plan(int64_t M, int H, int n, int k) {
  Plan pl;
  pl.nblk = (int)cdiv(n, 32);
  pl.qblocks = cdiv(M, kQueriesPerGroup);
  const int64_t base = pl.qblocks * 2 * H;
  int64_t s = cdiv(MPL_SCORE_TARGET_WGS, base);
  s = s < 1 ? 1 : s;
  s = s > kMaxSplits ? kMaxSplits : s;
  s = s > pl.nblk ? pl.nblk : s;
  pl.blk_per_split = (int)cdiv(pl.nblk, s);
  pl.splits = (int)cdiv(pl.nblk, pl.blk_per_split);
  pl.kmax = k <= 16 ? 16 : 32;
  const int p1 = pl.blk_per_split / MPL_PASS1_DIV;
  pl.pass1_blocks = std::min(pl.blk_per_split, std::max(MPL_PASS1_MIN, p1));
  return pl;
}

// Decode plans (score_topk_decode): M <= kDecodeMaxQ tokens and k <= 16,
// with fp16 scoring and no noise; a split is one workgroup's 64*WPG keys.
static bool decode_shape(int64_t M, int k) { return M >= 1 && M <= kDecodeMaxQ && k <= 16; }

static Plan make_decode_plan(int n) {
  Plan pl;
  pl.nblk = (int)cdiv(n, 32);
  pl.qblocks = 1;
  pl.blk_per_split = 2 * kDecodeWaves;
  pl.splits = (int)cdiv(pl.nblk, pl.blk_per_split);
  pl.kmax = 16;
  pl.pass1_blocks = 0;
  return pl;
}

// Workspace: the select scores with noise; per-split lists when split, and
// for k == 16 the lists of each reduction level (8 lists into one) until at
// most 8 remain for stage 2.
static int reduced_total(const Plan& pl, int k) {
  int tot = 0;
  for (int S = pl.splits; k == 16 && S > kMergeChunk; S = (int)cdiv(S, kMergeChunk)) tot += (int)cdiv(S, kMergeChunk);
  return tot;
}

static size_t ws_bytes(const Plan& pl, int64_t M, int H, int k, bool noise) {
  const size_t per = (size_t)M * 2 * H * k;
  if (pl.splits == 1) return noise ? per * 4 : 0;
  return per * (pl.splits + reduced_total(pl, k)) * (noise ? 3 : 2) * 4;
}

// Register-loaded keys cost up to 32 more VGPRs than LDS tiles; they are used
// where the kernel stays at the same occupancy without AGPRs (measured with
// -Rpass-analysis=kernel-resource-usage on gfx950).
template <typename T, int HP, bool NOISE, int KMAX>
constexpr bool direct_keys() {
  constexpr int vpl = KeyPack<T>::vectors_per_lane(HP);
  const bool occ1 = KMAX == 32 || (NOISE && vpl >= 8) || (!NOISE && vpl > 8);
  const bool occ3 = !NOISE && vpl == 2;
  return !occ1 && !occ3;
}
template <typename T, int HP, bool NOISE, int KMAX>
static void launch_stage1(const ScoreParams& sp, int64_t blocks, hipStream_t s) {
  constexpr bool D = direct_keys<T, HP, NOISE, KMAX>();
  if constexpr (!NOISE && short_fits<T, HP>(4)) {
    if (sp.blk_per_split <= 4) {
      score_topk_kernel<T, HP, NOISE, KMAX, false, 4><<<(unsigned)blocks, kScoreThreads, 0, s>>>(sp);
      return;
    }
  }
  if constexpr (!NOISE && short_fits<T, HP>(8)) {
    if (sp.blk_per_split <= 8) {
      score_topk_kernel<T, HP, NOISE, KMAX, false, 8><<<(unsigned)blocks, kScoreThreads, 0, s>>>(sp);
      return;
    }
  }
  score_topk_kernel<T, HP, NOISE, KMAX, D, 0><<<(unsigned)blocks, kScoreThreads, 0, s>>>(sp);
}

template <int HP>
static void launch_decode(const ScoreParams& sp, int64_t blocks, hipStream_t s) {
  const unsigned g = (unsigned)blocks;
  constexpr int W = kDecodeWaves;
  if (sp.M == 1) score_topk_decode<HP, 1, W><<<g, 64 * W, 0, s>>>(sp);
  else if (sp.M == 2) score_topk_decode<HP, 2, W><<<g, 64 * W, 0, s>>>(sp);
  else score_topk_decode<HP, 4, W><<<g, 64 * W, 0, s>>>(sp);
}

static int dispatch_decode(const ScoreParams& sp, int64_t blocks, int HP, hipStream_t s) {
  switch (HP) {
    case 16: launch_decode<16>(sp, blocks, s); break;
    case 32: launch_decode<32>(sp, blocks, s); break;
    case 64: launch_decode<64>(sp, blocks, s); break;
    case 128: launch_decode<128>(sp, blocks, s); break;
    default: return MPL_EUNSUPPORTED;
  }
  return MPL_OK;
}

template <typename T, int HP>
static void dispatch_noise_kmax(const ScoreParams& sp, int64_t blocks, bool noise, int kmax,
                                hipStream_t s) {
  if (noise) {
    if (kmax == 16) launch_stage1<T, HP, true, 16>(sp, blocks, s);
    else launch_stage1<T, HP, true, 32>(sp, blocks, s);
  } else {
    if (kmax == 16) launch_stage1<T, HP, false, 16>(sp, blocks, s);
    else launch_stage1<T, HP, false, 32>(sp, blocks, s);
  }
}

static int dispatch_stage1(const ScoreParams& sp, int64_t blocks, int score_dtype, int HP, bool noise,
                           int kmax, hipStream_t s) {
  if (score_dtype == MPL_F16) {
    switch (HP) {
      case 16: dispatch_noise_kmax<_Float16, 16>(sp, blocks, noise, kmax, s); break;
      case 32: dispatch_noise_kmax<_Float16, 32>(sp, blocks, noise, kmax, s); break;
      case 64: dispatch_noise_kmax<_Float16, 64>(sp, blocks, noise, kmax, s); break;
      case 128: dispatch_noise_kmax<_Float16, 128>(sp, blocks, noise, kmax, s); break;
      default: return MPL_EUNSUPPORTED;
    }
  } else {
    switch (HP) {
      case 8: dispatch_noise_kmax<float, 8>(sp, blocks, noise, kmax, s); break;
      case 16: dispatch_noise_kmax<float, 16>(sp, blocks, noise, kmax, s); break;
      case 32: dispatch_noise_kmax<float, 32>(sp, blocks, noise, kmax, s); break;
      case 64: dispatch_noise_kmax<float, 64>(sp, blocks, noise, kmax, s); break;
      case 128: dispatch_noise_kmax<float, 128>(sp, blocks, noise, kmax, s); break;
      default: return MPL_EUNSUPPORTED;
    }
  }
  return MPL_OK;
}

}  // namespace mpl

using namespace mpl;

// Scratch of the stage-1-only call beyond the selection's: with several
// splits and k != 16 the lists are combined by the pair kernel, whose slot
// outputs (flat_idx, slots, weights) then go to scratch.
static size_t topk_extra_bytes(const Plan& pl, int64_t M, int H, int k) {
  return (pl.splits > 1 && k != 16) ? (size_t)M * H * k * 3 * 4 : 0;
}

// The sizes cover every plan a call of these shapes may take (the decode
// plan depends on the scoring type and noise, which the size query lacks).
extern "C" size_t mpl_score_select_workspace_bytes(int64_t M, int H, int n, int half, int k) {
  (void)half;
  if (M <= 0 || H <= 0 || n <= 0 || k <= 0) return 0;
  size_t need = ws_bytes(make_plan(M, H, n, k), M, H, k, true);
  if (decode_shape(M, k)) need = std::max(need, ws_bytes(make_decode_plan(n), M, H, k, false));
  return need;
}

extern "C" size_t mpl_score_topk_workspace_bytes(int64_t M, int H, int n, int half, int k) {
  (void)half;
  if (M <= 0 || H <= 0 || n <= 0 || k <= 0) return 0;
  auto need = [&](const Plan& pl, bool noise) {
    return (ws_bytes(pl, M, H, k, noise) + 255) / 256 * 256 + topk_extra_bytes(pl, M, H, k);
  };
  size_t b = need(make_plan(M, H, n, k), true);
  if (decode_shape(M, k)) b = std::max(b, need(make_decode_plan(n), false));
  return b;
}

// Both entry points: stage 1 (+ the split-list reduction); with `pair`, stage
// 2 and the softmax as well.  Without `pair`, flat_idx/slots/weights are null.
// The value read fused into stage 2 (pair_read_k16), when the shapes allow:
// returns false (nothing launched) otherwise.
struct LookupRead {
  const void* values;
  int dtype;  // MPL_F16 or MPL_F32
  int d;
  int shuffle;
  float* out;
};

static bool launch_pair_read(const LookupRead& lr, const PairParams& pp, unsigned grid, hipStream_t s) {
  const int esz = lr.dtype == MPL_F16 ? 2 : 4;
  if (pp.H != 4 || pp.k != 16 || (lr.d * esz) % 16 != 0 || ((uintptr_t)lr.values % 16) != 0 ||
      ((uintptr_t)lr.out % 16) != 0)
    return false;
  ReadParams rp;
  rp.values = lr.values;
  rp.shuffle = lr.shuffle;
  rp.out = lr.out;
  const int VR = lr.d * esz / 16;
  const bool nt = (int64_t)pp.n * pp.n * lr.d * esz > kStreamTableBytes;
#define MPL_PR(V, vr)                                               \
  if (VR == vr) {                                                   \
    if (nt)                                                         \
      pair_read_k16<V, vr, true><<<grid, 256, 0, s>>>(pp, rp);      \
    else                                                            \
      pair_read_k16<V, vr, false><<<grid, 256, 0, s>>>(pp, rp);     \
    return true;                                                    \
  }
  if (lr.dtype == MPL_F16) {
    MPL_PR(_Float16, 16) MPL_PR(_Float16, 32) MPL_PR(_Float16, 64)
  } else {
    MPL_PR(float, 32) MPL_PR(float, 64)
  }
#undef MPL_PR
  return false;
}

// The value read fused into pair_wide_k16 (pair_wide_read_k16): same shape
// conditions as launch_pair_read; returns false (nothing launched) otherwise.
static bool launch_pair_wide_read(const LookupRead& lr, const PairParams& pp, hipStream_t s) {
  const int esz = lr.dtype == MPL_F16 ? 2 : 4;
  if (pp.H != 4 || pp.k != 16 || (lr.d * esz) % 16 != 0 || ((uintptr_t)lr.values % 16) != 0 ||
      ((uintptr_t)lr.out % 16) != 0)
    return false;
  ReadParams rp;
  rp.values = lr.values;
  rp.shuffle = lr.shuffle;
  rp.out = lr.out;
  const int VR = lr.d * esz / 16;
  const bool nt = (int64_t)pp.n * pp.n * lr.d * esz > kStreamTableBytes;
  const unsigned grid = (unsigned)pp.M;
#define MPL_PWR(V, vr)                                                   \
  if (VR == vr) {                                                        \
    if (nt)                                                              \
      pair_wide_read_k16<V, vr, true><<<grid, 1024, 0, s>>>(pp, rp);     \
    else                                                                 \
      pair_wide_read_k16<V, vr, false><<<grid, 1024, 0, s>>>(pp, rp);    \
    return true;                                                         \
  }
  if (lr.dtype == MPL_F16) {
    MPL_PWR(_Float16, 16) MPL_PWR(_Float16, 32) MPL_PWR(_Float16, 64)
  } else {
    MPL_PWR(float, 32) MPL_PWR(float, 64)
  }
#undef MPL_PWR
  return false;
}

// The decode stage 2 fused with the value read (pair_decode_read_k16): the
// conditions of launch_pair_read and one row group per lane (VR <= 64);
// returns false (nothing launched) otherwise.
static bool launch_pair_decode_read(const LookupRead& lr, const PairParams& pp, hipStream_t s) {
  const int esz = lr.dtype == MPL_F16 ? 2 : 4;
  if (pp.H != 4 || pp.k != 16 || pp.sel != nullptr || pp.S > kDecodeMaxSplits || (lr.d * esz) % 16 != 0 ||
      ((uintptr_t)lr.values % 16) != 0 || ((uintptr_t)lr.out % 16) != 0)
    return false;
  ReadParams rp;
  rp.values = lr.values;
  rp.shuffle = lr.shuffle;
  rp.out = lr.out;
  const int VR = lr.d * esz / 16;
  const bool nt = (int64_t)pp.n * pp.n * lr.d * esz > kStreamTableBytes;
  const unsigned grid = (unsigned)pp.M;
#define MPL_PDR(V, vr)                                                          \
  if (VR == vr) {                                                               \
    if (pp.S <= 32) {                                                           \
      if (nt)                                                                   \
        pair_decode_read_k16<V, vr, true, 32><<<grid, 1024, 0, s>>>(pp, rp);    \
      else                                                                      \
        pair_decode_read_k16<V, vr, false, 32><<<grid, 1024, 0, s>>>(pp, rp);   \
    } else {                                                                    \
      if (nt)                                                                   \
        pair_decode_read_k16<V, vr, true, 64><<<grid, 1024, 0, s>>>(pp, rp);    \
      else                                                                      \
        pair_decode_read_k16<V, vr, false, 64><<<grid, 1024, 0, s>>>(pp, rp);   \
    }                                                                           \
    return true;                                                                \
  }
  if (lr.dtype == MPL_F16) {
    MPL_PDR(_Float16, 16) MPL_PDR(_Float16, 32) MPL_PDR(_Float16, 64)
  } else {
    MPL_PDR(float, 32) MPL_PDR(float, 64)
  }
#undef MPL_PDR
  return false;
}

static int select_impl(const char* who, bool pair, const void* queries, int query_mode, float* q_len,
                       const void* packed_keys, int64_t M, int H, int n, int half, int k, int score_dtype,
                       const float* temperature, const float* gumbel, const float* noise_coef, void* workspace,
                       size_t workspace_bytes, int32_t* sub_idx, float* sub_scores, int32_t* flat_idx,
                       int32_t* slots, float* weights, void* stream, const LookupRead* read = nullptr,
                       bool* read_done = nullptr) {
  if (read_done != nullptr) *read_done = false;
  clear_error();
  MPL_REQUIRE(M >= 0 && H > 0 && n > 0 && half > 0 && k > 0, MPL_EINVAL,
              "%s: bad sizes M=%lld H=%d n=%d half=%d k=%d", who, (long long)M, H, n, half, k);
  MPL_REQUIRE(k <= n && k <= 32, MPL_EUNSUPPORTED, "%s: need k <= min(n, 32), got k=%d n=%d", who, k, n);
  MPL_REQUIRE(half <= 128, MPL_EUNSUPPORTED, "%s: half=%d > 128", who, half);
  MPL_REQUIRE(score_dtype != MPL_F16 || half % 8 == 0, MPL_EUNSUPPORTED,
              "%s: fp16 scoring needs half %% 8 == 0 (got %d); use MPL_F32", who, half);
  MPL_REQUIRE((int64_t)n * n < ((int64_t)1 << 31), MPL_EUNSUPPORTED, "%s: n*n must be < 2^31", who);
  MPL_REQUIRE(score_dtype == MPL_F16 || score_dtype == MPL_F32, MPL_EINVAL,
              "%s: score_dtype must be MPL_F16 or MPL_F32", who);
  if (M == 0) return MPL_OK;
  MPL_REQUIRE(queries && packed_keys && sub_idx && sub_scores && (!pair || (flat_idx && slots && weights)),
              MPL_EINVAL, "%s: null buffer", who);
  MPL_REQUIRE(temperature != nullptr && (gumbel == nullptr || noise_coef != nullptr), MPL_EINVAL,
              "%s: null temperature (or noise_coef with gumbel) device scalar", who);
  MPL_REQUIRE(query_mode == MPL_Q_NORMALIZED || query_mode == MPL_Q_RAW || query_mode == MPL_Q_RAW_SCALED,
              MPL_EINVAL, "%s: bad query_mode %d", who, query_mode);
  const bool noise = gumbel != nullptr;
  const bool decode = !noise && score_dtype == MPL_F16 && decode_shape(M, k);
  const Plan pl = decode ? make_decode_plan(n) : make_plan(M, H, n, k);
  const size_t sel_need = ws_bytes(pl, M, H, k, noise);
  const size_t extra = pair ? 0 : topk_extra_bytes(pl, M, H, k);
  const size_t extra_at = (sel_need + 255) / 256 * 256;
  const size_t need = extra ? extra_at + extra : sel_need;
  MPL_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr), MPL_EWORKSPACE,
              "%s: workspace of %zu bytes needed, %zu given", who, need, workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  const int HC = 2 * H;
  const size_t per = (size_t)M * HC * k;

  ScoreParams sp;
  sp.q_hat = queries;
  sp.q_len = query_mode == MPL_Q_NORMALIZED ? q_len : nullptr;
  sp.out_qlen = query_mode == MPL_Q_RAW_SCALED ? q_len : nullptr;
  sp.query_mode = query_mode;
  sp.packed = (const uint4*)packed_keys;
  sp.gumbel = gumbel;
  sp.T = temperature;
  sp.noise_coef = noise_coef;
  sp.noise_vec = noise && ((uintptr_t)gumbel & 15) == 0 && n % 4 == 0;
  sp.M = M;
  sp.HC = HC;
  sp.n = n;
  sp.half = half;
  sp.k = k;
  sp.nblk = pl.nblk;
  sp.splits = pl.splits;
  sp.blk_per_split = pl.blk_per_split;
  sp.pass1_blocks = pl.pass1_blocks;
  float* w = (float*)workspace;
  const size_t part = per * pl.splits;
  if (pl.splits == 1) {
    sp.out_clean = sub_scores;
    sp.out_idx = sub_idx;
    sp.out_sel = noise ? w : nullptr;
  } else {
    sp.out_clean = w;
    sp.out_idx = (int*)(w + part);
    sp.out_sel = noise ? w + 2 * part : nullptr;
  }
  const int HP = score_dtype == MPL_F16 ? KeyPack<_Float16>::padded_half(half) : KeyPack<float>::padded_half(half);
  const int64_t blocks = pl.qblocks * pl.splits * HC;
  int rc = decode ? dispatch_decode(sp, blocks, HP, s)
                  : dispatch_stage1(sp, blocks, score_dtype, HP, noise, pl.kmax, s);
  if (rc) {
    set_error("%s: unsupported padded half %d", who, HP);
    return rc;
  }
  rc = check_launch(pair ? "mpl_score_select(stage 1)" : "mpl_score_topk(stage 1)");
  if (rc) return rc;

  PairParams pp;
  pp.sel = sp.out_sel;
  pp.clean = sp.out_clean;
  pp.idx = sp.out_idx;
  pp.M = M;
  pp.H = H;
  pp.n = n;
  pp.k = k;
  pp.S = pl.splits;
  pp.sub_idx = sub_idx;
  pp.sub_scores = sub_scores;
  pp.flat_idx = flat_idx;
  pp.slots = slots;
  pp.weights = weights;
  // many splits (decode-sized batches): reduce the lists in parallel, eight
  // into one per level, so stage 2 merges at most 8 lists instead of a long
  // sequential chain
  if (pair && k == 16 && pp.S > kMergeChunk && pp.S <= kWideMaxSplits) {
    if (read != nullptr && pp.S <= kDecodeMaxSplits && launch_pair_decode_read(*read, pp, s)) {
      *read_done = true;
      return check_launch("mpl_lookup(decode stage 2 + value read)");
    }
    if (read != nullptr && M > 0 && launch_pair_wide_read(*read, pp, s)) {
      *read_done = true;
      return check_launch("mpl_lookup(wide stage 2 + value read)");
    }
    pair_wide_k16<<<(unsigned)(M * H), 256, 0, s>>>(pp);
    return check_launch("mpl_score_select(stage 2)");
  }
  float* r = w + (noise ? 3 : 2) * part;
  while (k == 16 && pp.S > kMergeChunk) {
    const int S2 = (int)cdiv(pp.S, kMergeChunk);
    const size_t part2 = per * S2;
    MergeParams mp;
    mp.sel = pp.sel;
    mp.clean = pp.clean;
    mp.idx = pp.idx;
    mp.rows = M * HC;
    mp.S = pp.S;
    mp.S2 = S2;
    mp.out_clean = r;
    mp.out_idx = (int*)(r + part2);
    mp.out_sel = noise ? r + 2 * part2 : nullptr;
    merge_splits_k16<<<(unsigned)cdiv(mp.rows * S2 * 16, 256), 256, 0, s>>>(mp);
    rc = check_launch("mpl_score_select(split merge)");
    if (rc) return rc;
    pp.sel = mp.out_sel;
    pp.clean = mp.out_clean;
    pp.idx = mp.out_idx;
    pp.S = S2;
    r += (noise ? 3 : 2) * part2;
  }
  if (!pair && pp.S == 1) return MPL_OK;  // stage 1 wrote sub_idx / sub_scores
  if (!pair && k == 16) {
    // the last reduction level writes the single list straight to the outputs
    MergeParams mp;
    mp.sel = pp.sel;
    mp.clean = pp.clean;
    mp.idx = pp.idx;
    mp.rows = M * HC;
    mp.S = pp.S;
    mp.S2 = 1;
    mp.out_clean = sub_scores;
    mp.out_idx = sub_idx;
    mp.out_sel = nullptr;
    merge_splits_k16<<<(unsigned)cdiv(mp.rows * 16, 256), 256, 0, s>>>(mp);
    return check_launch("mpl_score_topk(split merge)");
  }
  if (!pair) {  // k != 16 with splits: the pair kernel combines them; its slot outputs go to scratch
    char* x = (char*)workspace + extra_at;
    const size_t mhk = (size_t)M * H * k;
    pp.flat_idx = (int32_t*)x;
    pp.slots = (int32_t*)(x + mhk * 4);
    pp.weights = (float*)(x + mhk * 8);
  }
  const int G = k <= 16 ? 16 : 32;
  const unsigned g2 = (unsigned)cdiv(M * H * G, 256);
  if (k == 16 && read != nullptr && launch_pair_read(*read, pp, g2, s)) {
    *read_done = true;
    return check_launch("mpl_lookup(stage 2 + value read)");
  }
  if (k == 16) pair_kernel_k16<<<g2, 256, 0, s>>>(pp);
  else if (G == 16) pair_kernel<16><<<g2, 256, 0, s>>>(pp);
  else pair_kernel<32><<<g2, 256, 0, s>>>(pp);
  return check_launch(pair ? "mpl_score_select(stage 2)" : "mpl_score_topk(split lists)");
}

extern "C" int mpl_score_select(const void* queries, int query_mode, float* q_len, const void* packed_keys,
                                int64_t M, int H, int n, int half, int k, int score_dtype,
                                const float* temperature, const float* gumbel, const float* noise_coef,
                                void* workspace, size_t workspace_bytes, int32_t* sub_idx,
                                float* sub_scores, int32_t* flat_idx, int32_t* slots,
                                float* weights, void* stream) {
  return select_impl("mpl_score_select", true, queries, query_mode, q_len, packed_keys, M, H, n, half, k,
                     score_dtype, temperature, gumbel, noise_coef, workspace, workspace_bytes, sub_idx,
                     sub_scores, flat_idx, slots, weights, stream);
}

extern "C" int mpl_score_topk(const void* queries, int query_mode, float* q_len, const void* packed_keys,
                              int64_t M, int H, int n, int half, int k, int score_dtype, const float* temperature,
                              const float* gumbel, const float* noise_coef, void* workspace, size_t workspace_bytes,
                              int32_t* sub_idx, float* sub_scores, void* stream) {
  return select_impl("mpl_score_topk", false, queries, query_mode, q_len, packed_keys, M, H, n, half, k,
                     score_dtype, temperature, gumbel, noise_coef, workspace, workspace_bytes, sub_idx,
                     sub_scores, nullptr, nullptr, nullptr, stream);
}

extern "C" int mpl_lookup(const void* queries, int query_mode, float* q_len, const void* packed_keys, int64_t M,
                          int H, int n, int half, int k, int score_dtype, const float* temperature, const float* gumbel,
                          const float* noise_coef, void* workspace, size_t workspace_bytes, int32_t* sub_idx,
                          float* sub_scores, int32_t* flat_idx, int32_t* slots, float* weights,
                          const void* values, int values_dtype, int d, int shuffle_reads, float* out,
                          void* stream) {
  clear_error();
  MPL_REQUIRE(values_dtype == MPL_F16 || values_dtype == MPL_F32, MPL_EINVAL,
              "mpl_lookup: values_dtype must be MPL_F16 or MPL_F32");
  MPL_REQUIRE(d > 0, MPL_EINVAL, "mpl_lookup: bad d=%d", d);
  MPL_REQUIRE(M == 0 || (values != nullptr && out != nullptr), MPL_EINVAL, "mpl_lookup: null buffer");
  const LookupRead lr{values, values_dtype, d, shuffle_reads != 0, out};
  bool done = false;
  int rc = select_impl("mpl_lookup", true, queries, query_mode, q_len, packed_keys, M, H, n, half, k, score_dtype,
                       temperature, gumbel, noise_coef, workspace, workspace_bytes, sub_idx, sub_scores, flat_idx,
                       slots, weights, stream, &lr, &done);
  if (rc || done || M == 0) return rc;
  return mpl_gather_wsum(values, values_dtype, (int64_t)n * n, d, slots, weights, M, H * k, shuffle_reads,
                              out, stream);
}

// -------------------------------------------------- lookup without allocation
// mpl_lookup_static: mpl_lookup with the selection's scratch in `scratch`, a
// fixed array of kStaticScratchBytes on each GPU the library runs on (held
// until the process ends), so the caller passes no workspace.  Each call
// writes every byte of scratch it later reads (split lists, reduced lists,
// noisy select scores) before reading it, so nothing is cleared between
// calls.  Calls that overlap on one GPU share the array and race.
constexpr size_t kStaticScratchBytes = (size_t)32 << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];
static std::mutex g_scratch_mu;
static void* g_scratch_addr[kMaxDevices];

// Device address of the current device's copy of `scratch`.  In host code the
// array's name is only a handle; the address is looked up once per device,
// with that device current, and used from then on.
static int static_scratch(void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  MPL_REQUIRE(e == hipSuccess, MPL_EHIP, "mpl_lookup_static: hipGetDevice: %s", hipGetErrorString(e));
  MPL_REQUIRE(dev >= 0 && dev < kMaxDevices, MPL_EUNSUPPORTED, "mpl_lookup_static: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    MPL_REQUIRE(e == hipSuccess && p != nullptr, MPL_EHIP, "mpl_lookup_static: hipGetSymbolAddress: %s",
                hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return MPL_OK;
}

extern "C" size_t mpl_lookup_static_scratch_bytes(void) { return kStaticScratchBytes; }

extern "C" int mpl_lookup_static(const void* queries, int query_mode, float* q_len, const void* packed_keys,
                                 int64_t M, int H, int n, int half, int k, int score_dtype, const float* temperature,
                                 const float* gumbel, const float* noise_coef, int32_t* sub_idx, float* sub_scores,
                                 int32_t* flat_idx, int32_t* slots, float* weights, const void* values,
                                 int values_dtype, int d, int shuffle_reads, float* out, void* stream) {
  clear_error();
  const size_t need = mpl_score_select_workspace_bytes(M, H, n, half, k);
  MPL_REQUIRE(need <= kStaticScratchBytes, MPL_EWORKSPACE,
              "mpl_lookup_static: %lld tokens need %zu bytes of scratch, more than its fixed %zu; "
              "split the batch or call mpl_lookup with a workspace",
              (long long)M, need, kStaticScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    // the scratch is the current device's copy: the stream must be on that device
    int cur = -1;
    hipDevice_t sdev = -1;
    hipError_t e = hipGetDevice(&cur);
    MPL_REQUIRE(e == hipSuccess, MPL_EHIP, "mpl_lookup_static: hipGetDevice: %s", hipGetErrorString(e));
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    MPL_REQUIRE(e == hipSuccess, MPL_EHIP, "mpl_lookup_static: hipStreamGetDevice: %s", hipGetErrorString(e));
    MPL_REQUIRE((int)sdev == cur, MPL_EINVAL,
                "mpl_lookup_static: the stream belongs to device %d but device %d is current; make the stream's "
                "device current before the call",
                (int)sdev, cur);
    const int rc = static_scratch(&ws);
    if (rc) return rc;
  }
  return mpl_lookup(queries, query_mode, q_len, packed_keys, M, H, n, half, k, score_dtype, temperature, gumbel,
                    noise_coef, ws, need, sub_idx, sub_scores, flat_idx, slots, weights, values, values_dtype, d,
                    shuffle_reads, out, stream);
}
