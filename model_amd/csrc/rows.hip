// Sparse value gradients and row-wise optimizers of the memory pool
// (train.py:146-172, 395-399, 409-426).
//
// merge_rows: the gradient of a fetched row is the sum, over the fetches of
// that slot, of weight * dL/dout of the fetching token.  The reference
// materialises one contribution row per fetch and runs jnp.unique +
// segment_sum; here the (slot, fetch) pairs are sorted by slot with a stable
// LSD radix sort (8-bit digits), runs of equal slots become segments, and
// each segment's rows are summed in a fixed order straight from dL/dout, so
// the contribution rows never exist and no float atomics are used: the
// result is bitwise reproducible.
//
// Radix pass (three kernels): per-tile digit histograms laid out
// digit-major, one exclusive scan over them, and a stable scatter in which
// each wave ranks its 64 keys by digit with ballots (lanes of equal digit
// and lower lane id), waves of a tile are ordered through LDS counters, and
// tiles through the scanned histogram.
//
// Segmented sum: wave r owns sorted entries [r*128, r*128 + 128), loads
// their (fetch, segment, weight) once (two per lane) and walks them in order,
// the dL/dout rows of the next batch loading while the current batch is
// added.  A segment that lies inside the range is written as a finished row;
// the range's first and last segment, when they cross the range boundary,
// leave partial sums that a fix-up kernel (one wave per range: the segment
// that starts there) adds in range order.  Hot rows (Zipf-skewed routing)
// therefore spread over many waves without changing the summation order from
// run to run.
#include <math.h>

#include <algorithm>

#include "common.h"

namespace mpl {

constexpr int kSortThreads = 256;
constexpr int kSortRounds = 8;
constexpr int kSortTile = kSortThreads * kSortRounds;  // keys per tile
constexpr int kRangeLen = 128;                         // sorted entries per reduce wave
constexpr int kRowThreads = 256;                       // four rows (waves) per block

__device__ __forceinline__ uint64_t lanes_below(int lane) { return (1ull << lane) - 1ull; }

// Mask of the valid lanes whose BITS-bit digit equals this lane's.
template <int BITS>
__device__ __forceinline__ uint64_t digit_peers(uint32_t digit, bool valid) {
  uint64_t peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < BITS; ++b) {
    const bool bit = (digit >> b) & 1u;
    const uint64_t m = __ballot(bit);
    peers &= bit ? m : ~m;
  }
  return peers;
}

// ------------------------------------------------------------ radix sort
// Digits of BITS = 8, 9 or 10 bits (2^BITS bins), chosen per key width so
// that the passes are as few as possible (pool sizes up to 2^20: two passes).
// zero_out[0, zero_n), when not null, is cleared on the side (the per-slot
// fetch counts that the segment kernels fill in later).
template <int BITS>
__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const uint32_t* __restrict__ keys, int64_t n,
                                                                   int shift, uint32_t* __restrict__ hist,
                                                                   int64_t ntiles, float* __restrict__ zero_out,
                                                                   int64_t zero_n) {
  constexpr int BINS = 1 << BITS;
  __shared__ uint32_t h[BINS];
  const int tid = threadIdx.x;
  if (zero_out != nullptr)
    for (int64_t i = (int64_t)blockIdx.x * kSortThreads + tid; i < zero_n; i += (int64_t)gridDim.x * kSortThreads)
      zero_out[i] = 0.f;
  for (int i = tid; i < BINS; i += kSortThreads) h[i] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t i = base + r * kSortThreads + tid;
    if (i < n) atomicAdd(&h[(keys[i] >> shift) & (BINS - 1)], 1u);  // integer LDS counts: order-free
  }
  __syncthreads();
  for (int i = tid; i < BINS; i += kSortThreads) hist[(int64_t)i * ntiles + blockIdx.x] = h[i];
}

// Exclusive scan of each digit's row hist[digit][0, ntiles) (one workgroup
// per digit, chunks of 1024 tiles); the digit's total goes to totals[digit].
__global__ __launch_bounds__(1024) void digit_scan_kernel(uint32_t* __restrict__ hist, int64_t ntiles,
                                                          uint32_t* __restrict__ totals) {
  __shared__ uint32_t wsum[1024 / kWave];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  uint32_t* row = hist + (int64_t)blockIdx.x * ntiles;
  uint32_t carry = 0;
  for (int64_t c0 = 0; c0 < ntiles; c0 += 1024) {
    const int64_t i = c0 + tid;
    const uint32_t v = i < ntiles ? row[i] : 0u;
    uint32_t x = v;  // inclusive scan within the wave
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t y = __shfl_up(x, off);
      if (lane >= off) x += y;
    }
    if (lane == kWave - 1) wsum[wave] = x;
    __syncthreads();
    uint32_t before = carry;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    uint32_t chunk = 0;
    for (int w = 0; w < 1024 / kWave; ++w) chunk += wsum[w];
    if (i < ntiles) row[i] = before + x - v;
    carry += chunk;
    __syncthreads();
  }
  if (tid == 0) totals[blockIdx.x] = carry;
}

// Stable scatter of one radix pass.  vals_in == null means the identity
// (values = input positions).  hist_scan holds each digit's scan over tiles;
// the digits' starting offsets are the scan of `totals`, done here in LDS
// (thread t owns digits [t PER, t PER + PER)).
template <int BITS>
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, int64_t n, int shift, const uint32_t* __restrict__ hist_scan, int64_t ntiles,
    const uint32_t* __restrict__ totals) {
  constexpr int BINS = 1 << BITS;
  constexpr int PER = BINS / kSortThreads;  // digits per thread
  constexpr int WAVES = kSortThreads / kWave;
  static_assert(PER >= 1 && BINS % kWave == 0, "at least one digit per thread");
  __shared__ uint32_t tile_off[BINS];
  __shared__ uint32_t seen[BINS];  // keys of each digit in earlier rounds of this tile
  __shared__ uint32_t wave_cnt[WAVES][BINS];
  __shared__ uint32_t wsum[WAVES];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  {  // digit base = exclusive scan of the digit totals
    uint32_t t[PER];
    uint32_t own = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      t[j] = totals[tid * PER + j];
      own += t[j];
    }
    uint32_t x = own;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t y = __shfl_up(x, off);
      if (lane >= off) x += y;
    }
    if (lane == kWave - 1) wsum[wave] = x;
    __syncthreads();
    uint32_t run = x - own;
    for (int w = 0; w < wave; ++w) run += wsum[w];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int d = tid * PER + j;
      tile_off[d] = run + hist_scan[(int64_t)d * ntiles + blockIdx.x];
      seen[d] = 0;
      run += t[j];
    }
    __syncthreads();
  }
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t i = base + r * kSortThreads + tid;
    const bool valid = i < n;
    const uint32_t key = keys_in[valid ? i : 0];
    const uint32_t val = vals_in != nullptr ? vals_in[valid ? i : 0] : (uint32_t)i;
    const uint32_t digit = (key >> shift) & (BINS - 1);
    const uint64_t peers = digit_peers<BITS>(digit, valid);
    const uint32_t rank = (uint32_t)__popcll(peers & lanes_below(lane));
    // this wave's row of counts: zeroed and filled by the wave itself (its
    // LDS accesses complete in order), read by all after the barrier
#pragma unroll
    for (int j = 0; j < BINS / kWave; ++j) wave_cnt[wave][lane * (BINS / kWave) + j] = 0;
    if (valid && rank == 0) wave_cnt[wave][digit] = (uint32_t)__popcll(peers);
    __syncthreads();
    uint32_t before = 0;
    for (int w = 0; w < wave; ++w) before += wave_cnt[w][digit];
    if (valid) {
      const uint32_t pos = tile_off[digit] + seen[digit] + before + rank;
      keys_out[pos] = key;
      vals_out[pos] = val;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int d = tid * PER + j;
      uint32_t add = 0;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) add += wave_cnt[w][d];
      seen[d] += add;
    }
    __syncthreads();
  }
}

// --------------------------------------------------------------- segments
__device__ __forceinline__ bool seg_head(const uint32_t* s, int64_t i) { return i == 0 || s[i] != s[i - 1]; }

__global__ __launch_bounds__(kSortThreads) void seg_count_kernel(const uint32_t* __restrict__ s, int64_t n,
                                                                  uint32_t* __restrict__ tile_cnt) {
  __shared__ uint32_t c[kSortThreads / kWave];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  uint32_t cnt = 0;
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t i = base + r * kSortThreads + tid;
    cnt += (i < n && seg_head(s, i)) ? 1u : 0u;
  }
  for (int off = 32; off >= 1; off >>= 1) cnt += __shfl_xor(cnt, off);
  if ((tid & 63) == 0) c[tid >> 6] = cnt;
  __syncthreads();
  if (tid == 0) {
    uint32_t t = 0;
    for (int w = 0; w < kSortThreads / kWave; ++w) t += c[w];
    tile_cnt[blockIdx.x] = t;
  }
}

// Segment u starts at sorted position seg_start[u] and has slot uniq[u];
// seg_of[i] is the segment of position i.  Segment ids are clamped to
// cap - 1 (the capacity of uniq / seg_start): only ids outside
// [0, pool_size) can make more distinct values than that, and they then get
// wrong results, never out-of-bounds writes.  Each workgroup takes its
// tile's first segment id as the sum of the tile counts before it (no scan
// launch); workgroup 0 sums them all for *total, the number of segments.
__global__ __launch_bounds__(kSortThreads) void seg_write_kernel(const uint32_t* __restrict__ s, int64_t n,
                                                                  const uint32_t* __restrict__ tile_cnt,
                                                                  int64_t ntiles, uint32_t* __restrict__ total,
                                                                  int32_t* __restrict__ uniq,
                                                                  int32_t* __restrict__ seg_start,
                                                                  int32_t* __restrict__ seg_of, int64_t cap) {
  __shared__ uint32_t wave_cnt[kSortThreads / kWave];
  __shared__ uint32_t seen;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  uint32_t tb;
  {
    const int64_t lim = blockIdx.x == 0 ? ntiles : (int64_t)blockIdx.x;
    uint32_t acc = 0;
    for (int64_t j = tid; j < lim; j += kSortThreads) acc += tile_cnt[j];
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) wave_cnt[wave] = acc;
    __syncthreads();
    uint32_t sum = 0;
    for (int w = 0; w < kSortThreads / kWave; ++w) sum += wave_cnt[w];
    tb = blockIdx.x == 0 ? 0u : sum;
    if (blockIdx.x == 0 && tid == 0 && total != nullptr) *total = sum;
    if (tid == 0) seen = 0;
    __syncthreads();  // wave_cnt is reused below
  }
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t i = base + r * kSortThreads + tid;
    const bool valid = i < n;
    const bool head = valid && seg_head(s, i);
    const uint64_t heads = __ballot(head);
    if (lane == 0) wave_cnt[wave] = (uint32_t)__popcll(heads);
    __syncthreads();
    uint32_t before = seen;
    for (int w = 0; w < wave; ++w) before += wave_cnt[w];
    // inclusive count of heads up to this lane, minus one
    const uint32_t incl = before + (uint32_t)__popcll(heads & (lanes_below(lane) | (1ull << lane)));
    if (valid) {
      const uint32_t u = (uint32_t)min((int64_t)(tb + incl - 1u), cap - 1);
      seg_of[i] = (int32_t)u;
      if (head) {
        uniq[u] = (int32_t)s[i];
        seg_start[u] = (int32_t)i;
      }
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t t = 0;
      for (int w = 0; w < kSortThreads / kWave; ++w) t += wave_cnt[w];
      seen += t;
    }
    __syncthreads();
  }
}

// --------------------------------------------------------- segmented sum
// A row of d floats is nv vectors of W floats (W = 4 when d % 4 == 0, else
// 1); lane l owns vectors l, l+64, ...  Loads are clamped and zeroed after,
// so lanes past the row end hold zeros.
template <int W>
struct RowVec {
  float x[W];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < W; ++i) x[i] = 0.f;
  }
  __device__ __forceinline__ void load(const float* p, int64_t vec, bool in) {
    const int64_t o = (in ? vec : 0) * W;
    if (W == 4) {
      const float4 f = *(const float4*)(p + o);
      x[0] = f.x;
      x[W > 1 ? 1 : 0] = f.y;
      x[W > 2 ? 2 : 0] = f.z;
      x[W > 3 ? 3 : 0] = f.w;
    } else {
      x[0] = p[o];
    }
    if (!in) zero();
  }
  __device__ __forceinline__ void store(float* p, int64_t vec) const {
    if (W == 4) {
      *(float4*)(p + vec * W) = make_float4(x[0], x[W > 1 ? 1 : 0], x[W > 2 ? 2 : 0], x[W > 3 ? 3 : 0]);
    } else {
      p[vec] = x[0];
    }
  }
  __device__ __forceinline__ void fma_add(float w, const RowVec& r) {
#pragma unroll
    for (int i = 0; i < W; ++i) x[i] += w * r.x[i];
  }
  __device__ __forceinline__ void add(const RowVec& r) {
#pragma unroll
    for (int i = 0; i < W; ++i) x[i] += r.x[i];
  }
  __device__ __forceinline__ float sq() const {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < W; ++i) s += x[i] * x[i];
    return s;
  }
};

template <int W, int VPL>
__device__ __forceinline__ float wave_sq(const RowVec<W> (&a)[VPL]) {
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) s += a[v].sq();
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  return s;
}

// Thread 0 of workgroup 0 also finishes the segment table (seg_start[U] =
// n, num_unique = U, U clamped to cap), which the fix-up launches read.
template <int W, int VPL>
__global__ __launch_bounds__(kRowThreads) void seg_reduce_kernel(
    const uint32_t* __restrict__ sorted_p, const int32_t* __restrict__ seg_of,
    const float* __restrict__ weights, const float* __restrict__ g, int fpt, int nv, int64_t n,
    float* __restrict__ rows, float* __restrict__ row_sq, float* __restrict__ partial,
    const uint32_t* __restrict__ num_seg, int32_t* __restrict__ seg_start, int32_t* __restrict__ num_unique,
    int64_t cap) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const uint32_t U = (uint32_t)min((int64_t)*num_seg, cap);
    seg_start[U] = (int32_t)n;
    *num_unique = (int32_t)U;
  }
  const int64_t r = ((int64_t)blockIdx.x * kRowThreads + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t r0 = r * kRangeLen;
  if (r0 >= n) return;
  const int64_t r1 = r0 + kRangeLen < n ? r0 + kRangeLen : n;

  RowVec<W> acc[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) acc[v].zero();
  int cur = seg_of[r0];
  bool first = true;
  // Segments are runs of equal ids in sorted order, so only the range's
  // first segment can start before r0 and only its last can end at or after
  // r1: a segment lies inside the range unless it is the first and position
  // r0 - 1 belongs to it, or the last and position r1 does.  Both tests are
  // read here once, so emitting a segment needs no load of its bounds.
  const int seg_first = cur;
  const int seg_last = seg_of[r1 - 1];
  const bool first_open = r0 > 0 && seg_of[r0 > 0 ? r0 - 1 : 0] == seg_first;
  const bool last_open = r1 < n && seg_of[r1 < n ? r1 : n - 1] == seg_last;
  auto emit = [&](int seg) {
    const bool open = (seg == seg_first && first_open) || (seg == seg_last && last_open);
    if (!open) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int c = lane + kWave * v;
        if (c < nv) acc[v].store(rows, (int64_t)seg * nv + c);
      }
      const float sq = wave_sq<W, VPL>(acc);
      if (lane == 0) row_sq[seg] = sq;
    } else {
      const int slot = first ? 0 : 1;
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int c = lane + kWave * v;
        if (c < nv) acc[v].store(partial, (r * 2 + slot) * nv + c);
      }
    }
  };
  // The range's (fetch, segment, weight) entries are loaded once, two per
  // lane (coalesced), and broadcast with shuffles; the g rows of the next
  // batch of B entries load while the current batch is accumulated (B rows
  // of VPL vectors per buffer, so the registers do not grow with the width).
  // At 8,192 tokens x 64 fetches of d = 256 the merge took 151 / 137 / 140 /
  // 141 us with B = 8 / 4 / 2 / 1: the g rows come from L2 and the Infinity
  // Cache (512 MB per call), and deeper batches only add cache pressure.
  static_assert(kRangeLen == 2 * kWave, "two entries per lane");
  constexpr int B = VPL >= 4 ? 1 : 4 / VPL;
  uint32_t pe[2];
  int se[2];
  float we[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t e = r0 + h * kWave + lane;
    const int64_t ec = e < r1 ? e : r1 - 1;
    pe[h] = sorted_p[ec];
    se[h] = seg_of[ec];
    we[h] = weights != nullptr ? weights[pe[h]] : 1.f;
  }
  const int len = (int)(r1 - r0);
  auto fetch = [&](int i, RowVec<W> (&row)[B][VPL], int* sg, float* ww) __attribute__((always_inline)) {
    const int h = i >= kWave;  // wave-uniform: a batch never straddles the halves (B divides 64)
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int src = (i + j) & (kWave - 1);
      const uint32_t pp = (uint32_t)__shfl((int)(h ? pe[1] : pe[0]), src);
      sg[j] = __shfl(h ? se[1] : se[0], src);
      ww[j] = __shfl(h ? we[1] : we[0], src);
      const int64_t t = pp / (uint32_t)fpt;
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int c = lane + kWave * v;
        row[j][v].load(g, t * nv + c, c < nv);
      }
    }
  };
  auto consume = [&](int i, const RowVec<W> (&row)[B][VPL], const int* sg, const float* ww)
                     __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < B; ++j) {
      if (i + j < len) {
        if (sg[j] != cur) {
          emit(cur);
#pragma unroll
          for (int v = 0; v < VPL; ++v) acc[v].zero();
          cur = sg[j];
          first = false;
        }
#pragma unroll
        for (int v = 0; v < VPL; ++v) acc[v].fma_add(ww[j], row[j][v]);
      }
    }
  };
  RowVec<W> ra[B][VPL], rb[B][VPL];
  int sa[B], sb[B];
  float wa[B], wb[B];
  fetch(0, ra, sa, wa);
  for (int i = 0; i < len; i += 2 * B) {
    if (i + B < len) fetch(i + B, rb, sb, wb);
    consume(i, ra, sa, wa);
    if (i + B >= len) break;
    if (i + 2 * B < len) fetch(i + 2 * B, ra, sa, wa);
    consume(i + B, rb, sb, wb);
  }
  emit(cur);
}

// Rows [U, cap): slot pool_size, zero row, zero norm (jnp.unique's
// fill_value and segment_sum's empty segments, train.py:166-172), by the
// workgroups [fix_blocks, gridDim) of the fix-up launch.
// slot_counts (when not null, cleared beforehand): the length of each
// segment of an id inside [0, pool_size), at that id.  Segment u ends where
// u + 1 starts (seg_start[U] = n, written by the reduce kernel).
__device__ __forceinline__ void pad_rows(const uint32_t* __restrict__ num_seg, int64_t cap, int d, int64_t pool_size,
                                         int32_t* __restrict__ uniq, float* __restrict__ rows,
                                         float* __restrict__ row_sq, int64_t t0, int64_t stride,
                                         const int32_t* __restrict__ seg_start, float* __restrict__ slot_counts) {
  const int64_t U = *num_seg;
  if (slot_counts != nullptr) {
    const int64_t Uc = U < cap ? U : cap;
    for (int64_t u = t0; u < Uc; u += stride) {
      const uint32_t id = (uint32_t)uniq[u];
      if (id < (uint64_t)pool_size) slot_counts[id] = (float)(seg_start[u + 1] - seg_start[u]);
    }
  }
  for (int64_t u = U + t0; u < cap; u += stride) {
    uniq[u] = (int32_t)pool_size;
    row_sq[u] = 0.f;
  }
  if (rows == nullptr) return;  // padding rows left unwritten
  if ((d & 3) == 0) {
    float4* r4 = (float4*)(rows + U * d);
    const int64_t n4 = (cap - U) * (d / 4);
    for (int64_t i = t0; i < n4; i += stride) r4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    float* r = rows + U * d;
    const int64_t n1 = (cap - U) * d;
    for (int64_t i = t0; i < n1; i += stride) r[i] = 0.f;
  }
}

// Segments that cross range boundaries are finished in two levels, so that a
// hot row spanning hundreds of ranges is summed by many waves at once in a
// fixed order.  Level 1 (seg_fix_chunks_kernel): for a crossing segment
// spanning ranges [ra, rb], the ranges are cut into chunks of kFixChunk
// starting at ra; the wave of a chunk's first range adds the chunk's
// partial rows in range order into chunk[head][which] (which = 1 when the
// segment starts in that range, so that the two crossing segments a range
// can head, the one it continues and the one it starts, use different
// rows).  Level 2 (seg_fixup_kernel): the wave of range ra adds the chunk
// rows in chunk order and writes the segment's row and squared norm.  A
// segment of one chunk (at most kFixChunk ranges: every crossing segment of
// near-uniform routing) skips level 1: level 2 adds its partial rows in
// range order itself, the same sum with the same bits, since level 2's
// zero-started sum of one chunk row returns that row (a sum started at +0
// is never -0).  Rows of segments inside one range were written by
// seg_reduce_kernel.  The level-2 launch also pads rows [U, cap) with its
// last workgroups.
constexpr int kFixChunk = 32;

// PB rows of partial-style storage (stride 2 rows per index) added in
// index order: rows idx(b), b = 0 .. count-1, PB loads in flight.
template <int W, int VPL, int PB, typename Idx>
__device__ __forceinline__ void add_rows(const float* __restrict__ src, int nv, int lane, int64_t count, Idx idx,
                                         RowVec<W> (&acc)[VPL]) {
  for (int64_t b0 = 0; b0 < count; b0 += PB) {
    RowVec<W> p[PB][VPL];
#pragma unroll
    for (int b = 0; b < PB; ++b) {
      const int64_t row = idx(b0 + b < count ? b0 + b : count - 1);
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int c = lane + kWave * v;
        p[b][v].load(src, row * nv + c, c < nv);
      }
    }
#pragma unroll
    for (int b = 0; b < PB; ++b)
      if (b0 + b < count)
#pragma unroll
        for (int v = 0; v < VPL; ++v) acc[v].add(p[b][v]);
  }
}

template <int W, int VPL>
__global__ __launch_bounds__(kRowThreads) void seg_fix_chunks_kernel(const int32_t* __restrict__ seg_start,
                                                                      const int32_t* __restrict__ seg_of, int64_t n,
                                                                      int nv, const float* __restrict__ partial,
                                                                      float* __restrict__ chunk) {
  const int64_t r = ((int64_t)blockIdx.x * kRowThreads + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t r0 = r * kRangeLen;
  if (r0 >= n) return;
  const int64_t r1 = r0 + kRangeLen < n ? r0 + kRangeLen : n;
  const int uf = seg_of[r0], ul = seg_of[r1 - 1];
  constexpr int PB = VPL >= 8 ? 4 : 32 / VPL;
  for (int t = 0; t < 2; ++t) {  // the segment this range continues, then the one it ends with
    if (t == 1 && ul == uf) break;
    const int u = t == 0 ? uf : ul;
    const int64_t s0 = seg_start[u], s1 = seg_start[u + 1];
    const int64_t ra = s0 / kRangeLen, rb = (s1 - 1) / kRangeLen;
    // inside one range, one chunk (level 2 adds its partials), or not a chunk head here
    if (ra == rb || rb - ra < kFixChunk || (r - ra) % kFixChunk != 0) continue;
    const int slot_a = s0 == ra * kRangeLen ? 0 : 1;
    const int64_t count = (rb - r + 1) < kFixChunk ? (rb - r + 1) : kFixChunk;
    RowVec<W> acc[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) acc[v].zero();
    add_rows<W, VPL, PB>(partial, nv, lane, count,
                         [&](int64_t b) { const int64_t q = r + b; return q * 2 + (q == ra ? slot_a : 0); }, acc);
    const int64_t out = r * 2 + (r == ra ? 1 : 0);
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int c = lane + kWave * v;
      if (c < nv) acc[v].store(chunk, out * nv + c);
    }
  }
}

template <int W, int VPL>
__global__ __launch_bounds__(kRowThreads) void seg_fixup_kernel(const int32_t* __restrict__ seg_start,
                                                                 const int32_t* __restrict__ seg_of, int64_t n,
                                                                 int nv, const float* __restrict__ partial,
                                                                 const float* __restrict__ chunk,
                                                                 float* __restrict__ rows,
                                                                 float* __restrict__ row_sq, int64_t fix_blocks,
                                                                 const uint32_t* __restrict__ num_seg, int64_t cap,
                                                                 int64_t pool_size, int32_t* __restrict__ uniq,
                                                                 int zero_padding, float* __restrict__ slot_counts) {
  if ((int64_t)blockIdx.x >= fix_blocks) {
    pad_rows(num_seg, cap, nv * W, pool_size, uniq, zero_padding ? rows : nullptr, row_sq,
             ((int64_t)blockIdx.x - fix_blocks) * kRowThreads + threadIdx.x,
             ((int64_t)gridDim.x - fix_blocks) * kRowThreads, seg_start, slot_counts);
    return;
  }
  const int64_t r = ((int64_t)blockIdx.x * kRowThreads + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t r0 = r * kRangeLen;
  if (r0 >= n) return;
  const int64_t r1 = r0 + kRangeLen < n ? r0 + kRangeLen : n;
  const int u = seg_of[r1 - 1];
  const int64_t s0 = seg_start[u], s1 = seg_start[u + 1];
  const int64_t ra = s0 / kRangeLen, rb = (s1 - 1) / kRangeLen;
  if (ra == rb || ra != r) return;  // inside one range, or another wave's segment
  RowVec<W> acc[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) acc[v].zero();
  constexpr int PB = VPL >= 8 ? 4 : 32 / VPL;
  if (rb - ra < kFixChunk) {  // one chunk: its partial rows, in range order (level 1 skipped it)
    const int slot_a = s0 == ra * kRangeLen ? 0 : 1;
    add_rows<W, VPL, PB>(partial, nv, lane, rb - ra + 1,
                         [&](int64_t b) { const int64_t q = ra + b; return q * 2 + (q == ra ? slot_a : 0); }, acc);
  } else {
    const int64_t nchunks = (rb - ra) / kFixChunk + 1;
    add_rows<W, VPL, PB>(chunk, nv, lane, nchunks,
                         [&](int64_t j) { const int64_t h = ra + j * kFixChunk; return h * 2 + (j == 0 ? 1 : 0); },
                         acc);
  }
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = lane + kWave * v;
    if (c < nv) acc[v].store(rows, (int64_t)u * nv + c);
  }
  const float sq = wave_sq<W, VPL>(acc);
  if (lane == 0) row_sq[u] = sq;
}

__global__ void seg_finish_kernel(const uint32_t* __restrict__ num_seg, int64_t n, int32_t* __restrict__ seg_start,
                                  int32_t* __restrict__ num_unique, int64_t cap) {
  const uint32_t U = (uint32_t)min((int64_t)*num_seg, cap);
  seg_start[U] = (int32_t)n;
  *num_unique = (int32_t)U;
}

__global__ void store_zero_kernel(int32_t* p) { *p = 0; }

__global__ __launch_bounds__(256) void zero_floats_kernel(float* __restrict__ x, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) x[i] = 0.f;
}

// ---------------------------------------------------------- global norm
// train.py:395-396 over the rows: sum of row_sq in a fixed order (fp64), then
// gnorm = sqrt(rest + sum) and scale = min(1, clip / (gnorm + 1e-6)).
// Stage 1: block b sums the contiguous chunk b; stage 2 sums the chunks.
constexpr int kSumBlocks = 256;

__device__ __forceinline__ double block_sum_f64(double s, double* part) {
  const int tid = threadIdx.x;
  part[tid] = s;
  __syncthreads();
  for (int off = blockDim.x / 2; off >= 1; off >>= 1) {
    if (tid < off) part[tid] += part[tid + off];
    __syncthreads();
  }
  return part[0];
}

__global__ __launch_bounds__(256) void sum_chunks_kernel(const float* __restrict__ x, int64_t n,
                                                         double* __restrict__ chunk_sums) {
  __shared__ double part[256];
  const int64_t per = cdiv(n, kSumBlocks);
  const int64_t b0 = (int64_t)blockIdx.x * per;
  const int64_t b1 = b0 + per < n ? b0 + per : n;
  double s = 0.0;
  for (int64_t i = b0 + threadIdx.x; i < b1; i += 256) s += (double)x[i];
  const double t = block_sum_f64(s, part);
  if (threadIdx.x == 0) chunk_sums[blockIdx.x] = t;
}

__global__ __launch_bounds__(256) void clip_finish_kernel(const double* __restrict__ chunk_sums,
                                                          const float* __restrict__ rest_sq, float clip,
                                                          float* __restrict__ out) {
  __shared__ double part[256];
  const double t = block_sum_f64(chunk_sums[threadIdx.x], part);
  if (threadIdx.x == 0) {
    const double total = t + (rest_sq != nullptr ? (double)*rest_sq : 0.0);
    const float gnorm = (float)sqrt(total);
    out[0] = fminf(1.f, clip / (gnorm + 1e-6f));
    out[1] = gnorm;
  }
}

// Sum of squares over up to kSqMaxBufs buffers, read as one array in order
// (buffer 0's elements, then buffer 1's, ...): block b sums chunk b of that
// array in fp64, the finish adds the chunks in order.  Same two-stage shape
// as the clip's row sum, so the result is bitwise reproducible.
constexpr int kSqMaxBufs = 8;
struct SqBufs {
  const float* x[kSqMaxBufs];
  int64_t end[kSqMaxBufs];  // exclusive prefix ends of the buffers in the joined array
  int count;
  unsigned plain;  // bit j: buffer j holds squares already (summed as they are)
};

__global__ __launch_bounds__(256) void sum_sq_chunks_kernel(SqBufs bufs, double* __restrict__ chunk_sums) {
  __shared__ double part[256];
  const int64_t total = bufs.end[bufs.count - 1];
  const int64_t per = cdiv(total, kSumBlocks);
  const int64_t b0 = (int64_t)blockIdx.x * per;
  const int64_t b1 = b0 + per < total ? b0 + per : total;
  double s = 0.0;
  int64_t start = 0;
  for (int j = 0; j < bufs.count; ++j) {
    const int64_t lo = b0 > start ? b0 : start;
    const int64_t hi = b1 < bufs.end[j] ? b1 : bufs.end[j];
    const float* __restrict__ x = bufs.x[j];
    if ((bufs.plain >> j) & 1u) {
      for (int64_t i = lo + threadIdx.x; i < hi; i += 256) s += (double)x[i - start];
    } else {
      for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
        const double v = (double)x[i - start];
        s += v * v;
      }
    }
    start = bufs.end[j];
  }
  const double t = block_sum_f64(s, part);
  if (threadIdx.x == 0) chunk_sums[blockIdx.x] = t;
}

__global__ __launch_bounds__(256) void sum_finish_kernel(const double* __restrict__ chunk_sums,
                                                         const float* __restrict__ add, float* __restrict__ out) {
  __shared__ double part[256];
  const double t = block_sum_f64(chunk_sums[threadIdx.x], part);
  if (threadIdx.x == 0) out[0] = (float)(t + (add != nullptr ? (double)*add : 0.0));
}

// ---------------------------------------------------------- optimizers
// One wave per row, grid-stride over the cap rows (a fixed grid: most of the
// cap rows are padding when routing is skewed).  A row of d elements is nv
// vectors of W (4 when d % 4 == 0, else 1); lane l owns vectors l, l+64, ...
constexpr int kOptBlocks = 2048;

template <typename V, int W>
struct TableVec;
template <>
struct TableVec<float, 4> {
  __device__ static void load(const float* p, float* x) {
    const float4 f = *(const float4*)p;
    x[0] = f.x; x[1] = f.y; x[2] = f.z; x[3] = f.w;
  }
  __device__ static void store(float* p, const float* x) { *(float4*)p = make_float4(x[0], x[1], x[2], x[3]); }
};
template <>
struct TableVec<_Float16, 4> {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  __device__ static void load(const _Float16* p, float* x) {
    const h4 h = *(const h4*)p;
    x[0] = (float)h[0]; x[1] = (float)h[1]; x[2] = (float)h[2]; x[3] = (float)h[3];
  }
  __device__ static void store(_Float16* p, const float* x) {
    h4 h;
    h[0] = (_Float16)x[0]; h[1] = (_Float16)x[1]; h[2] = (_Float16)x[2]; h[3] = (_Float16)x[3];
    *(h4*)p = h;
  }
};
template <typename V>
struct TableVec<V, 1> {
  __device__ static void load(const V* p, float* x) { x[0] = (float)*p; }
  __device__ static void store(V* p, const float* x) { *p = (V)x[0]; }
};

// One wave per touched row, two rows in flight: the lanes first fetch the
// ids of the wave's next 64 rows (one load instead of one per row), then each
// iteration issues both rows' gradient, master and accumulator loads before
// any arithmetic, so the loads of a row do not wait for the previous row.
template <typename V, int W, int VPL>
__global__ __launch_bounds__(kRowThreads) void row_adagrad_kernel(V* __restrict__ values, float* __restrict__ master,
                                                                   float* __restrict__ acc,
                                                                   const int32_t* __restrict__ uniq,
                                                                   const float* __restrict__ rows, int64_t cap, int d,
                                                                   int64_t N, float lr,
                                                                   const float* __restrict__ grad_scale) {
  // rows in flight per wave: four for rows of up to 256 fp32 (one vector per
  // lane), one for very wide rows.  With 2,048 workgroups, 71.5k touched
  // rows of d = 256 update in 47.8 us (51.0 us with two rows and 1,024
  // workgroups; non-temporal row loads were slower, 51.6 us).
  constexpr int R = VPL >= 16 ? 1 : (VPL == 1 ? 4 : 2);
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * (kRowThreads / kWave);
  const int64_t wid = ((int64_t)blockIdx.x * kRowThreads + threadIdx.x) >> 6;
  const int nv = d / W;
  const float sc = grad_scale != nullptr ? *grad_scale : 1.f;
  for (int64_t base = wid; base < cap; base += kWave * nw) {
    const int64_t uj = base + lane * nw;
    const int sj = uj < cap ? uniq[uj] : -1;
    for (int it = 0; it < kWave; it += R) {
      if (base + it * nw >= cap) break;  // wave-uniform
      int64_t us[R], ss[R];
      bool ok[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        us[r] = base + (it + r) * nw;
        ss[r] = __shfl(sj, it + r);
        ok[r] = us[r] < cap && ss[r] >= 0 && ss[r] < N;  // padding (mode="drop")
      }
      float g[R][VPL][W], x[R][VPL][W], a0[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        a0[r] = ok[r] ? acc[ss[r]] : 0.f;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          const int c = lane + kWave * v;
          if (ok[r] && c < nv) {
            TableVec<float, W>::load(rows + us[r] * d + (int64_t)c * W, g[r][v]);
            if (VPL == 1) {  // wider rows load the table after the reduction (registers)
              const int64_t o = ss[r] * d + (int64_t)c * W;
              if (master != nullptr) TableVec<float, W>::load(master + o, x[r][v]);
              else TableVec<V, W>::load(values + o, x[r][v]);
            }
          }
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (!ok[r]) continue;  // wave-uniform
        float sq = 0.f;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          const int c = lane + kWave * v;
          if (c < nv) {
#pragma unroll
            for (int i = 0; i < W; ++i) {
              g[r][v][i] *= sc;
              sq += g[r][v][i] * g[r][v][i];
            }
          }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) sq += __shfl_xor(sq, off);
        const float a = a0[r] + sq / (float)d;
        const float step = lr / (sqrtf(a) + 1e-8f);
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          const int c = lane + kWave * v;
          if (c < nv) {
            const int64_t o = ss[r] * d + (int64_t)c * W;
            if (VPL != 1) {
              if (master != nullptr) TableVec<float, W>::load(master + o, x[r][v]);
              else TableVec<V, W>::load(values + o, x[r][v]);
            }
#pragma unroll
            for (int i = 0; i < W; ++i) x[r][v][i] += -step * g[r][v][i];
            if (master != nullptr) TableVec<float, W>::store(master + o, x[r][v]);
            TableVec<V, W>::store(values + o, x[r][v]);
          }
        }
        if (lane == 0) acc[ss[r]] = a;
      }
    }
  }
}

// train.py:417-426 (c1 = 1 - b1^n, c2 = 1 - b2^n with n = step + 1).
template <typename V, int W, int VPL>
__global__ __launch_bounds__(kRowThreads) void row_adam_kernel(V* __restrict__ values, float* __restrict__ master,
                                                                float* __restrict__ m1, float* __restrict__ m2,
                                                                const int32_t* __restrict__ uniq,
                                                                const float* __restrict__ rows, int64_t cap, int d,
                                                                int64_t N, float lr, float c1, float c2,
                                                                const float* __restrict__ grad_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * (kRowThreads / kWave);
  const int nv = d / W;
  const float sc = grad_scale != nullptr ? *grad_scale : 1.f;
  // train.py:421-422 writes (1 - ADAM_B1) and (1 - ADAM_B2) with Python
  // floats: computed in double and rounded once to fp32 (0.1f, 0.001f), not
  // 1.f - 0.9f (0.100000024f) and 1.f - 0.999f (0.00100004673f, 5e-5 off)
  const float b1 = 0.9f, b2 = 0.999f, ob1 = (float)(1.0 - 0.9), ob2 = (float)(1.0 - 0.999), eps = 1e-8f;
  constexpr int R = VPL >= 16 ? 1 : 2;  // rows in flight per wave, as in row_adagrad_kernel
  const int64_t wid = ((int64_t)blockIdx.x * kRowThreads + threadIdx.x) >> 6;
  for (int64_t base = wid; base < cap; base += kWave * nw) {
    const int64_t uj = base + lane * nw;
    const int sj = uj < cap ? uniq[uj] : -1;
    for (int it = 0; it < kWave; it += R) {
      if (base + it * nw >= cap) break;  // wave-uniform
      int64_t us[R], ss[R];
      bool ok[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        us[r] = base + (it + r) * nw;
        ss[r] = __shfl(sj, it + r);
        ok[r] = us[r] < cap && ss[r] >= 0 && ss[r] < N;
      }
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int c = lane + kWave * v;
        if (c >= nv) continue;
        float g[R][W], m[R][W], q[R][W], x[R][W];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (!ok[r]) continue;
          const int64_t o = ss[r] * d + (int64_t)c * W;
          TableVec<float, W>::load(rows + us[r] * d + (int64_t)c * W, g[r]);
          TableVec<float, W>::load(m1 + o, m[r]);
          TableVec<float, W>::load(m2 + o, q[r]);
          if (master != nullptr) TableVec<float, W>::load(master + o, x[r]);
          else TableVec<V, W>::load(values + o, x[r]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (!ok[r]) continue;
          const int64_t o = ss[r] * d + (int64_t)c * W;
#pragma unroll
          for (int i = 0; i < W; ++i) {
            const float gi = g[r][i] * sc;
            m[r][i] = b1 * m[r][i] + ob1 * gi;
            q[r][i] = b2 * q[r][i] + ob2 * gi * gi;
            x[r][i] += -lr * (m[r][i] / c1) / (sqrtf(q[r][i] / c2) + eps);
          }
          TableVec<float, W>::store(m1 + o, m[r]);
          TableVec<float, W>::store(m2 + o, q[r]);
          if (master != nullptr) TableVec<float, W>::store(master + o, x[r]);
          TableVec<V, W>::store(values + o, x[r]);
        }
      }
    }
  }
}

// ------------------------------------------------------------ host side
struct MergeLayout {
  int64_t ntiles, nranges, cap;
  int passes, digit_bits;
  size_t keys[2], vals[2], hist, tile_cnt, counters, totals, seg_start, seg_of, partial, chunk, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static MergeLayout merge_layout(int64_t P, int d, int64_t pool_size) {
  MergeLayout L;
  L.ntiles = cdiv(P, kSortTile);
  L.nranges = cdiv(P, kRangeLen);
  L.cap = P < pool_size ? P : pool_size;
  int bits = 0;
  while (bits < 62 && ((int64_t)1 << bits) < pool_size) ++bits;
  // fewest passes of at most 10 bits, each digit at least 8 bits wide
  L.passes = bits <= 10 ? 1 : (bits + 9) / 10;
  L.digit_bits = std::max(8, (int)cdiv(bits, L.passes));
  const int64_t nfl = d;  // partial rows: d floats
  size_t o = 0;
  for (int b = 0; b < 2; ++b) {
    L.keys[b] = o;
    o += align256((size_t)P * 4);
    L.vals[b] = o;
    o += align256((size_t)P * 4);
  }
  L.hist = o;
  o += align256(((size_t)1 << L.digit_bits) * L.ntiles * 4);
  L.tile_cnt = o;
  o += align256((size_t)L.ntiles * 4);
  L.counters = o;  // [0]: segment count
  o += 256;
  L.totals = o;  // digit totals of a radix pass
  o += align256(((size_t)1 << L.digit_bits) * 4);
  L.seg_start = o;
  o += align256((size_t)(L.cap + 1) * 4);
  L.seg_of = o;
  o += align256((size_t)P * 4);
  L.partial = o;
  o += align256((size_t)L.nranges * 2 * nfl * 4);
  L.chunk = o;  // first-level fix-up rows, indexed like the partial rows
  o += align256((size_t)L.nranges * 2 * nfl * 4);
  L.total = o;
  return L;
}

template <int W, int VPL>
static void launch_reduce(const uint32_t* sp, int32_t* seg_of, int32_t* seg_start, const float* weights,
                          const float* g, int fpt, int nv, int64_t P, float* rows, float* row_sq, float* partial,
                          float* chunk, const MergeLayout& L, const uint32_t* nseg, int64_t pool_size, int32_t* uniq,
                          int32_t* num_unique, int zero_padding, float* slot_counts, hipStream_t s) {
  const unsigned b1 = (unsigned)cdiv(L.nranges, kRowThreads / kWave);
  seg_reduce_kernel<W, VPL><<<b1, kRowThreads, 0, s>>>(sp, seg_of, weights, g, fpt, nv, P, rows, row_sq, partial,
                                                       nseg, seg_start, num_unique, L.cap);
  seg_fix_chunks_kernel<W, VPL><<<b1, kRowThreads, 0, s>>>(seg_start, seg_of, P, nv, partial, chunk);
  seg_fixup_kernel<W, VPL><<<b1 + 1024, kRowThreads, 0, s>>>(seg_start, seg_of, P, nv, partial, chunk, rows, row_sq, b1,
                                                             nseg, L.cap, pool_size, uniq, zero_padding,
                                                             slot_counts);
}

template <int W>
static void dispatch_reduce(const uint32_t* sp, int32_t* seg_of, int32_t* seg_start, const float* weights,
                            const float* g, int fpt, int nv, int64_t P, float* rows, float* row_sq, float* partial,
                            float* chunk, const MergeLayout& L, const uint32_t* nseg, int64_t pool_size,
                            int32_t* uniq, int32_t* num_unique, int zero_padding, float* slot_counts,
                            hipStream_t s) {
  const int vpl = (int)cdiv(nv, kWave);
#define MPL_REDUCE(V)                                                                                               \
  launch_reduce<W, V>(sp, seg_of, seg_start, weights, g, fpt, nv, P, rows, row_sq, partial, chunk, L, nseg,      \
                      pool_size, uniq, num_unique, zero_padding, slot_counts, s)
  if (vpl <= 1) MPL_REDUCE(1);
  else if (vpl <= 2) MPL_REDUCE(2);
  else if (vpl <= 4) MPL_REDUCE(4);
  else if (vpl <= 8) MPL_REDUCE(8);
  else MPL_REDUCE(16);
#undef MPL_REDUCE
}

}  // namespace mpl

using namespace mpl;

// LSD radix sort of the slots (positions as payload), then the segments of
// equal slots: uniq[u], seg_start[u] (seg_start[U] = P), seg_of[i] of sorted
// position i, num_unique = U.  The workspace is laid out by merge_layout().
struct Segments {
  const uint32_t* pos;  // original fetch position of each sorted entry
  int32_t* seg_start;
  int32_t* seg_of;
  uint32_t* nseg;
};

// finish = false leaves seg_start[U] and num_unique to the caller's next
// kernel (seg_reduce_kernel does it for mpl_merge_rows).
static Segments sort_segments(const uint32_t* slots, int64_t P, const MergeLayout& L, char* ws, int32_t* uniq,
                              int32_t* num_unique, bool finish, hipStream_t s, float* zero_out = nullptr,
                              int64_t zero_n = 0) {
  uint32_t* keys[2] = {(uint32_t*)(ws + L.keys[0]), (uint32_t*)(ws + L.keys[1])};
  uint32_t* vals[2] = {(uint32_t*)(ws + L.vals[0]), (uint32_t*)(ws + L.vals[1])};
  uint32_t* hist = (uint32_t*)(ws + L.hist);
  uint32_t* tile_cnt = (uint32_t*)(ws + L.tile_cnt);
  uint32_t* nseg = (uint32_t*)(ws + L.counters);
  uint32_t* totals = (uint32_t*)(ws + L.totals);
  int32_t* seg_start = (int32_t*)(ws + L.seg_start);
  int32_t* seg_of = (int32_t*)(ws + L.seg_of);
  const unsigned nt = (unsigned)L.ntiles;
  const uint32_t* kin = slots;
  const uint32_t* vin = nullptr;
  int cur = 0;
  for (int pass = 0; pass < L.passes; ++pass) {
    const int shift = L.digit_bits * pass;
#define MPL_RADIX(B)                                                                                        \
  radix_hist_kernel<B><<<nt, kSortThreads, 0, s>>>(kin, P, shift, hist, L.ntiles, pass == 0 ? zero_out : nullptr, \
                                                   zero_n);                                                       \
  digit_scan_kernel<<<1u << B, 1024, 0, s>>>(hist, L.ntiles, totals);                                       \
  radix_scatter_kernel<B><<<nt, kSortThreads, 0, s>>>(kin, vin, keys[cur], vals[cur], P, shift, hist, L.ntiles, \
                                                      totals)
    if (L.digit_bits <= 8) {
      MPL_RADIX(8);
    } else if (L.digit_bits == 9) {
      MPL_RADIX(9);
    } else {
      MPL_RADIX(10);
    }
#undef MPL_RADIX
    kin = keys[cur];
    vin = vals[cur];
    cur ^= 1;
  }
  seg_count_kernel<<<nt, kSortThreads, 0, s>>>(kin, P, tile_cnt);
  seg_write_kernel<<<nt, kSortThreads, 0, s>>>(kin, P, tile_cnt, L.ntiles, nseg, uniq, seg_start, seg_of, L.cap);
  if (finish) seg_finish_kernel<<<1, 1, 0, s>>>(nseg, P, seg_start, num_unique, L.cap);
  return Segments{vin, seg_start, seg_of, nseg};
}

// inverse[pos[i]] = seg_of[i]; uniq[u] = pool_size for num_unique <= u < len.
__global__ __launch_bounds__(256) void unique_finish_kernel(const uint32_t* __restrict__ pos,
                                                            const int32_t* __restrict__ seg_of, int64_t P,
                                                            const int32_t* __restrict__ num_unique,
                                                            int64_t pool_size, int32_t* __restrict__ uniq,
                                                            int32_t* __restrict__ inverse) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= P) return;
  inverse[pos[i]] = seg_of[i];
  if (i >= *num_unique) uniq[i] = (int32_t)pool_size;
}

extern "C" size_t mpl_unique_slots_workspace_bytes(int64_t P, int64_t pool_size) {
  if (P <= 0 || pool_size <= 0) return 0;
  return merge_layout(P, 4, pool_size > P ? pool_size : P).total;
}

extern "C" int mpl_unique_slots(const int32_t* slots, int64_t P, int64_t pool_size, void* workspace,
                                size_t workspace_bytes, int32_t* uniq, int32_t* inverse, int32_t* num_unique,
                                void* stream) {
  clear_error();
  MPL_REQUIRE(P >= 0 && pool_size > 0, MPL_EINVAL, "mpl_unique_slots: bad sizes P=%lld pool_size=%lld",
              (long long)P, (long long)pool_size);
  MPL_REQUIRE(P < ((int64_t)1 << 31) && pool_size < ((int64_t)1 << 31), MPL_EUNSUPPORTED,
              "mpl_unique_slots: P and pool_size must be < 2^31");
  MPL_REQUIRE(num_unique != nullptr, MPL_EINVAL, "mpl_unique_slots: null num_unique");
  hipStream_t s = (hipStream_t)stream;
  if (P == 0) {
    store_zero_kernel<<<1, 1, 0, s>>>(num_unique);
    return check_launch("mpl_unique_slots");
  }
  MPL_REQUIRE(slots && uniq && inverse, MPL_EINVAL, "mpl_unique_slots: null buffer");
  // segments are counted against P, not min(P, pool_size): any input, even
  // ids outside [0, pool_size), stays inside the [P] buffers
  const MergeLayout L = merge_layout(P, 4, pool_size > P ? pool_size : P);
  MPL_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, MPL_EWORKSPACE,
              "mpl_unique_slots: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
  const Segments sg = sort_segments((const uint32_t*)slots, P, L, (char*)workspace, uniq, num_unique, true, s);
  unique_finish_kernel<<<(unsigned)cdiv(P, 256), 256, 0, s>>>(sg.pos, sg.seg_of, P, num_unique, pool_size, uniq,
                                                              inverse);
  return check_launch("mpl_unique_slots");
}

extern "C" size_t mpl_merge_rows_workspace_bytes(int64_t P, int d, int64_t pool_size) {
  if (P <= 0 || d <= 0 || pool_size <= 0) return 0;
  return merge_layout(P, d, pool_size).total;
}

static int merge_rows_impl(const int32_t* slots, const float* weights, int64_t P, int fetches_per_token,
                           const float* g, int d, int64_t pool_size, void* workspace, size_t workspace_bytes,
                           int32_t* uniq, float* rows, float* row_sq, int32_t* num_unique, int zero_padding,
                           float* slot_counts, void* stream) {
  MPL_REQUIRE(P >= 0 && fetches_per_token > 0 && d > 0 && pool_size > 0, MPL_EINVAL,
              "mpl_merge_rows: bad sizes P=%lld fetches_per_token=%d d=%d pool_size=%lld", (long long)P,
              fetches_per_token, d, (long long)pool_size);
  MPL_REQUIRE(P < ((int64_t)1 << 31) && pool_size < ((int64_t)1 << 31), MPL_EUNSUPPORTED,
              "mpl_merge_rows: P and pool_size must be < 2^31");
  MPL_REQUIRE(d <= 16 * kWave, MPL_EUNSUPPORTED, "mpl_merge_rows: d must be <= 1024, got %d", d);
  hipStream_t s = (hipStream_t)stream;
  if (P == 0) {
    MPL_REQUIRE(num_unique != nullptr, MPL_EINVAL, "mpl_merge_rows: null num_unique");
    store_zero_kernel<<<1, 1, 0, s>>>(num_unique);  // a kernel, not a memset: safe under graph capture
    if (slot_counts != nullptr) zero_floats_kernel<<<(unsigned)std::min<int64_t>(cdiv(pool_size, 256), 4096), 256, 0, s>>>(slot_counts, pool_size);
    return check_launch("mpl_merge_rows");
  }
  MPL_REQUIRE(slots && g && uniq && rows && row_sq && num_unique, MPL_EINVAL, "mpl_merge_rows: null buffer");
  const MergeLayout L = merge_layout(P, d, pool_size);
  MPL_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, MPL_EWORKSPACE,
              "mpl_merge_rows: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
  char* ws = (char*)workspace;
  const Segments sg = sort_segments((const uint32_t*)slots, P, L, ws, uniq, num_unique, false, s, slot_counts,
                                    slot_counts != nullptr ? pool_size : 0);
  int rc = check_launch("mpl_merge_rows(sort)");
  if (rc) return rc;
  const uint32_t* vin = sg.pos;
  int32_t* seg_start = sg.seg_start;
  int32_t* seg_of = sg.seg_of;
  uint32_t* nseg = sg.nseg;
  float* partial = (float*)(ws + L.partial);
  float* chunk = (float*)(ws + L.chunk);
  if (d % 4 == 0)
    dispatch_reduce<4>(vin, seg_of, seg_start, weights, g, fetches_per_token, d / 4, P, rows, row_sq, partial, chunk,
                       L, nseg, pool_size, uniq, num_unique, zero_padding, slot_counts, s);
  else
    dispatch_reduce<1>(vin, seg_of, seg_start, weights, g, fetches_per_token, d, P, rows, row_sq, partial, chunk, L,
                       nseg, pool_size, uniq, num_unique, zero_padding, slot_counts, s);
  return check_launch("mpl_merge_rows(reduce)");
}

extern "C" int mpl_merge_rows(const int32_t* slots, const float* weights, int64_t P, int fetches_per_token,
                              const float* g, int d, int64_t pool_size, void* workspace, size_t workspace_bytes,
                              int32_t* uniq, float* rows, float* row_sq, int32_t* num_unique, int zero_padding,
                              void* stream) {
  clear_error();
  return merge_rows_impl(slots, weights, P, fetches_per_token, g, d, pool_size, workspace, workspace_bytes, uniq,
                         rows, row_sq, num_unique, zero_padding, nullptr, stream);
}

extern "C" int mpl_merge_rows_counts(const int32_t* slots, const float* weights, int64_t P, int fetches_per_token,
                                     const float* g, int d, int64_t pool_size, void* workspace,
                                     size_t workspace_bytes, int32_t* uniq, float* rows, float* row_sq,
                                     int32_t* num_unique, int zero_padding, float* slot_counts, void* stream) {
  clear_error();
  MPL_REQUIRE(slot_counts != nullptr, MPL_EINVAL, "mpl_merge_rows_counts: null slot_counts");
  return merge_rows_impl(slots, weights, P, fetches_per_token, g, d, pool_size, workspace, workspace_bytes, uniq,
                         rows, row_sq, num_unique, zero_padding, slot_counts, stream);
}

extern "C" size_t mpl_clip_scale_workspace_bytes() { return kSumBlocks * sizeof(double); }

extern "C" int mpl_clip_scale(const float* row_sq, int64_t cap, const float* rest_sq, float grad_clip,
                              float* scale_gnorm, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  MPL_REQUIRE(cap >= 0 && scale_gnorm != nullptr && (cap == 0 || row_sq != nullptr), MPL_EINVAL,
              "mpl_clip_scale: bad arguments");
  MPL_REQUIRE(workspace != nullptr && workspace_bytes >= kSumBlocks * sizeof(double), MPL_EWORKSPACE,
              "mpl_clip_scale: workspace of %zu bytes needed", (size_t)kSumBlocks * sizeof(double));
  hipStream_t s = (hipStream_t)stream;
  sum_chunks_kernel<<<kSumBlocks, 256, 0, s>>>(row_sq, cap, (double*)workspace);
  clip_finish_kernel<<<1, 256, 0, s>>>((const double*)workspace, rest_sq, grad_clip, scale_gnorm);
  return check_launch("mpl_clip_scale");
}

extern "C" int mpl_clip_scale_dense(const float* row_sq, int64_t cap, const float* const* x, const int64_t* n,
                                    int count, float grad_clip, float* scale_gnorm, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  clear_error();
  MPL_REQUIRE(cap >= 0 && scale_gnorm != nullptr && (cap == 0 || row_sq != nullptr), MPL_EINVAL,
              "mpl_clip_scale_dense: bad arguments");
  MPL_REQUIRE(count >= 0 && count < kSqMaxBufs && (count == 0 || (x && n)), MPL_EINVAL,
              "mpl_clip_scale_dense: bad dense buffers (count %d, at most %d)", count, kSqMaxBufs - 1);
  MPL_REQUIRE(workspace != nullptr && workspace_bytes >= kSumBlocks * sizeof(double), MPL_EWORKSPACE,
              "mpl_clip_scale_dense: workspace of %zu bytes needed", (size_t)kSumBlocks * sizeof(double));
  SqBufs b{};
  int64_t total = 0;
  int used = 0;
  if (cap > 0) {
    total = cap;
    b.x[0] = row_sq;
    b.end[0] = total;
    b.plain = 1u;
    used = 1;
  }
  for (int j = 0; j < count; ++j) {
    MPL_REQUIRE(n[j] >= 0 && (n[j] == 0 || x[j] != nullptr), MPL_EINVAL,
                "mpl_clip_scale_dense: buffer %d: bad size or null", j);
    if (n[j] == 0) continue;
    total += n[j];
    b.x[used] = x[j];
    b.end[used] = total;
    ++used;
  }
  if (used == 0) {
    b.x[0] = nullptr;
    b.end[0] = 0;
    used = 1;
  }
  b.count = used;
  hipStream_t s = (hipStream_t)stream;
  sum_sq_chunks_kernel<<<kSumBlocks, 256, 0, s>>>(b, (double*)workspace);
  clip_finish_kernel<<<1, 256, 0, s>>>((const double*)workspace, nullptr, grad_clip, scale_gnorm);
  return check_launch("mpl_clip_scale_dense");
}

extern "C" size_t mpl_sum_squares_workspace_bytes() { return kSumBlocks * sizeof(double); }

extern "C" int mpl_sum_squares(const float* const* x, const int64_t* n, int count, const float* add, float* out,
                               void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  MPL_REQUIRE(count >= 0 && count <= kSqMaxBufs && out != nullptr && (count == 0 || (x && n)), MPL_EINVAL,
              "mpl_sum_squares: bad arguments (count %d, at most %d buffers)", count, kSqMaxBufs);
  MPL_REQUIRE(workspace != nullptr && workspace_bytes >= kSumBlocks * sizeof(double), MPL_EWORKSPACE,
              "mpl_sum_squares: workspace of %zu bytes needed", (size_t)kSumBlocks * sizeof(double));
  SqBufs b{};
  int64_t total = 0;
  int used = 0;
  for (int j = 0; j < count; ++j) {
    MPL_REQUIRE(n[j] >= 0 && (n[j] == 0 || x[j] != nullptr), MPL_EINVAL, "mpl_sum_squares: buffer %d: bad size or null", j);
    if (n[j] == 0) continue;
    total += n[j];
    b.x[used] = x[j];
    b.end[used] = total;
    ++used;
  }
  if (used == 0) {  // an empty sum: out = add (or 0), one element, still a kernel
    b.x[0] = nullptr;
    b.end[0] = 0;
    used = 1;
  }
  b.count = used;
  hipStream_t s = (hipStream_t)stream;
  sum_sq_chunks_kernel<<<kSumBlocks, 256, 0, s>>>(b, (double*)workspace);
  sum_finish_kernel<<<1, 256, 0, s>>>((const double*)workspace, add, out);
  return check_launch("mpl_sum_squares");
}

extern "C" int mpl_row_adagrad(void* values, int values_dtype, float* master, float* acc, const int32_t* uniq,
                               const float* rows, int64_t cap, int d, int64_t pool_size, float lr,
                               const float* grad_scale, void* stream) {
  clear_error();
  MPL_REQUIRE(cap >= 0 && d > 0 && pool_size > 0, MPL_EINVAL, "mpl_row_adagrad: bad sizes");
  MPL_REQUIRE(values_dtype == MPL_F16 || values_dtype == MPL_F32, MPL_EINVAL,
              "mpl_row_adagrad: values_dtype must be MPL_F16 or MPL_F32");
  if (cap == 0) return MPL_OK;
  MPL_REQUIRE(values && acc && uniq && rows, MPL_EINVAL, "mpl_row_adagrad: null buffer");
  const unsigned b = (unsigned)std::min<int64_t>(kOptBlocks, cdiv(cap, kRowThreads / kWave));
  hipStream_t s = (hipStream_t)stream;
  const bool vec = d % 4 == 0;
  const int nv = vec ? d / 4 : d;
  const int vpl = (int)cdiv(nv, kWave);
  MPL_REQUIRE(vpl <= 16, MPL_EUNSUPPORTED, "mpl_row_adagrad: d must be <= 1024");
#define MPL_AG(V, W, P)                                                                                         \
  row_adagrad_kernel<V, W, P><<<b, kRowThreads, 0, s>>>((V*)values, master, acc, uniq, rows, cap, d, pool_size, \
                                                        lr, grad_scale)
#define MPL_AG_V(V, W)                     \
  if (vpl <= 1) MPL_AG(V, W, 1);           \
  else if (vpl <= 4) MPL_AG(V, W, 4);      \
  else MPL_AG(V, W, 16);
  if (values_dtype == MPL_F16) {
    if (vec) { MPL_AG_V(_Float16, 4) } else { MPL_AG_V(_Float16, 1) }
  } else {
    if (vec) { MPL_AG_V(float, 4) } else { MPL_AG_V(float, 1) }
  }
#undef MPL_AG_V
#undef MPL_AG
  return check_launch("mpl_row_adagrad");
}

extern "C" int mpl_row_adam(void* values, int values_dtype, float* master, float* m, float* v, const int32_t* uniq,
                            const float* rows, int64_t cap, int d, int64_t pool_size, float lr, int step,
                            const float* grad_scale, void* stream) {
  clear_error();
  MPL_REQUIRE(cap >= 0 && d > 0 && pool_size > 0 && step >= 0, MPL_EINVAL, "mpl_row_adam: bad sizes");
  MPL_REQUIRE(values_dtype == MPL_F16 || values_dtype == MPL_F32, MPL_EINVAL,
              "mpl_row_adam: values_dtype must be MPL_F16 or MPL_F32");
  if (cap == 0) return MPL_OK;
  MPL_REQUIRE(values && m && v && uniq && rows, MPL_EINVAL, "mpl_row_adam: null buffer");
  const float n = (float)(step + 1);
  const float c1 = 1.f - powf(0.9f, n);
  const float c2 = 1.f - powf(0.999f, n);
  const unsigned b = (unsigned)std::min<int64_t>(kOptBlocks, cdiv(cap, kRowThreads / kWave));
  hipStream_t s = (hipStream_t)stream;
  const bool vec = d % 4 == 0;
  const int nv = vec ? d / 4 : d;
  const int vpl = (int)cdiv(nv, kWave);
  MPL_REQUIRE(vpl <= 16, MPL_EUNSUPPORTED, "mpl_row_adam: d must be <= 1024");
#define MPL_AD(V, W, P)                                                                                           \
  row_adam_kernel<V, W, P><<<b, kRowThreads, 0, s>>>((V*)values, master, m, v, uniq, rows, cap, d, pool_size, lr, \
                                                     c1, c2, grad_scale)
#define MPL_AD_V(V, W)                     \
  if (vpl <= 1) MPL_AD(V, W, 1);           \
  else if (vpl <= 4) MPL_AD(V, W, 4);      \
  else MPL_AD(V, W, 16);
  if (values_dtype == MPL_F16) {
    if (vec) { MPL_AD_V(_Float16, 4) } else { MPL_AD_V(_Float16, 1) }
  } else {
    if (vec) { MPL_AD_V(float, 4) } else { MPL_AD_V(float, 1) }
  }
#undef MPL_AD_V
#undef MPL_AD
  return check_launch("mpl_row_adam");
}
