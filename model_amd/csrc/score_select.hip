// Product-key selection: cosine scoring on MFMA fused with the exact stage-1
// top-k (memory.py:149-164), then stage-2 top-k over the k*k candidates and
// the routing softmax (memory.py:167-178).
//
// Stage 1 (score_topk_kernel).  A workgroup owns 128 queries (two waves of
// 64) of one codebook hc = h*2 + c and one split of the n sub-keys.  Key
// blocks of 32 stream through LDS (double buffered); each wave computes a
// 32-key x 64-query score tile with two 32x32 MFMA chains, then swaps register
// halves across lanes (v_permlane32_swap) so that lane l owns query l with
// all 32 scores of the block.  Each lane keeps its query's running top-k as a
// sorted register list and a threshold (its k-th best).  Scores above the
// threshold are appended to a per-lane LDS candidate buffer; when any lane's
// buffer is nearly full the wave merges buffers into the lists (sorted
// insertion, strict '>' so an equal later key never displaces an earlier
// one).  Keys are visited in increasing index order, which makes the order
// (score desc, index asc) of lax.top_k fall out of the insertion rule.  The
// scores never leave registers/LDS.
//
// Without routing noise the selection runs on the raw cosine: scores are
// cos*T(*q_len) with positive per-query factors, so the order is the same up
// to ties created by the rounding of that product (near-ties).
//
// Stage 2 (stage2_kernel).  One thread per (token, head): merges the split
// lists of each codebook, then walks the k*k candidate grid in frontier order
// (row pointers; at step s only rows <= s can hold the next best), selecting
// by (select sum desc, flat index rank_a*k+rank_b asc) as memory.py:171, and
// finishes with the softmax of the clean slot scores (memory.py:178).
#include <limits.h>
#include <math.h>

#include "common.h"
#include "layout.h"

namespace mpl {

constexpr int kCand = 24;         // per-lane candidate buffer (entries)
constexpr int kScoreThreads = 128;  // two waves per workgroup
constexpr int kMaxSplits = 16;

struct ScoreParams {
  const float* q_hat;   // [M, HC, half]
  const float* q_len;   // [M, HC] or null
  const uint4* packed;  // packed keys
  const float* gumbel;  // [M, HC, n] or null
  float T, noise_coef;
  int64_t M;
  int HC, n, half, k, nblk, splits, blk_per_split;
  float* out_sel;    // [splits, M, HC, k] (may be null when no noise and splits == 1)
  float* out_clean;  // [splits, M, HC, k]
  int* out_idx;      // [splits, M, HC, k]
};

template <typename T>
struct Mfma;

template <>
struct Mfma<_Float16> {
  typedef half8 Op;
  __device__ static f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  // B operand for chunk c: dims 16c + 8*(lane/32) + [0,8) of query row q.
  __device__ static Op load_q(const float* q, bool valid, int half, int c, int lane) {
    Op o;
    const int d0 = 16 * c + 8 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (valid && d0 + i < half) ? (_Float16)q[d0 + i] : (_Float16)0.f;
    return o;
  }
  __device__ static Op from_vec(uint4 u, int) { return __builtin_bit_cast(half8, u); }
};

template <>
struct Mfma<float> {
  typedef float Op;
  __device__ static f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static Op load_q(const float* q, bool valid, int half, int c, int lane) {
    const int d = 2 * c + (lane >> 5);
    return (valid && d < half) ? q[d] : 0.f;
  }
  __device__ static Op from_vec(uint4 u, int e) {
    const unsigned w = e == 0 ? u.x : e == 1 ? u.y : e == 2 ? u.z : u.w;
    return __uint_as_float(w);
  }
};

// Sorted (descending) register list; insertion keeps earlier entries ahead
// of equal later ones.
template <int KMAX, bool NOISE>
struct TopList {
  float v[KMAX];
  int id[KMAX];
  float cl[NOISE ? KMAX : 1];

  __device__ void init() {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      v[j] = -INFINITY;
      id[j] = INT_MAX;
      if (NOISE) cl[j] = -INFINITY;
    }
  }
  __device__ void insert(float x, int xi, float xc) {
    bool c[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) c[j] = x > v[j];
#pragma unroll
    for (int j = KMAX - 1; j >= 1; --j) {
      v[j] = c[j - 1] ? v[j - 1] : (c[j] ? x : v[j]);
      id[j] = c[j - 1] ? id[j - 1] : (c[j] ? xi : id[j]);
      if (NOISE) cl[j] = c[j - 1] ? cl[j - 1] : (c[j] ? xc : cl[j]);
    }
    v[0] = c[0] ? x : v[0];
    id[0] = c[0] ? xi : id[0];
    if (NOISE) cl[0] = c[0] ? xc : cl[0];
  }
  __device__ float kth(int k) const {
    float t = v[0];
#pragma unroll
    for (int j = 1; j < KMAX; ++j) t = (j == k - 1) ? v[j] : t;
    return t;
  }
};

template <typename T, int HP, bool NOISE, int KMAX>
__global__ __launch_bounds__(kScoreThreads) void score_topk_kernel(ScoreParams p) {
  constexpr int VPL = KeyPack<T>::vectors_per_lane(HP);   // 16-B vectors per lane per block
  constexpr int OPV = KeyPack<T>::kOpsPerVec;
  constexpr int NCH = VPL * OPV;                          // MFMA chunks per block
  constexpr int TILE = VPL * kWave;                       // uint4 per key block
  constexpr int PRE = (TILE + kScoreThreads - 1) / kScoreThreads;
  typedef typename Mfma<T>::Op Op;

  __shared__ uint4 tiles[2][TILE];
  __shared__ float cs_[2][kCand][kWave];
  __shared__ int ci_[2][kCand][kWave];
  __shared__ float cc_[NOISE ? 2 : 1][NOISE ? kCand : 1][kWave];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int hc = blockIdx.x % p.HC;
  const int split = (blockIdx.x / p.HC) % p.splits;
  const int64_t qb = blockIdx.x / (p.HC * p.splits);
  const int64_t q0 = qb * kScoreThreads + wave * kWave;
  const int b_begin = split * p.blk_per_split;
  const int b_end = min(p.nblk, b_begin + p.blk_per_split);

  // B operands: set s holds queries q0 + 32*s + (lane % 32).
  Op qop[2][NCH];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int64_t qi = q0 + 32 * s + (lane & 31);
    const bool ok = qi < p.M;
    const float* qrow = p.q_hat + (ok ? (qi * p.HC + hc) * (int64_t)p.half : 0);
#pragma unroll
    for (int c = 0; c < NCH; ++c) qop[s][c] = Mfma<T>::load_q(qrow, ok, p.half, c, lane);
  }

  // Lane state: after the half swap lane l owns query q0 + l.
  const int64_t my_q = q0 + lane;
  const bool valid = my_q < p.M;
  const float ql = (p.q_len != nullptr && valid) ? p.q_len[my_q * p.HC + hc] : 1.f;
  const float* grow = NOISE && valid ? p.gumbel + (my_q * p.HC + hc) * (int64_t)p.n : nullptr;
  TopList<KMAX, NOISE> top;
  top.init();
  float thr = valid ? -INFINITY : INFINITY;
  int cnt = 0;

  auto flush = [&]() {
    for (int e = 0; e < kCand; ++e) {
      if (__ballot(e < cnt) == 0) break;
      const float x = e < cnt ? cs_[wave][e][lane] : -INFINITY;
      const int xi = ci_[wave][e][lane];
      const float xc = NOISE ? cc_[NOISE ? wave : 0][NOISE ? e : 0][lane] : 0.f;
      top.insert(x, xi, xc);
    }
    cnt = 0;
    if (valid) thr = top.kth(p.k);
  };

  const uint4* kbase_ptr = p.packed + (int64_t)hc * p.nblk * TILE;
  if (b_begin < b_end) {
#pragma unroll
    for (int i = 0; i < PRE; ++i) {
      const int t = tid + i * kScoreThreads;
      if (t < TILE) tiles[0][t] = kbase_ptr[(int64_t)b_begin * TILE + t];
    }
  }
  __syncthreads();

  for (int b = b_begin; b < b_end; ++b) {
    const int cur = (b - b_begin) & 1;
    const bool has_next = b + 1 < b_end;
    uint4 pre[PRE];
    if (has_next) {
#pragma unroll
      for (int i = 0; i < PRE; ++i) {
        const int t = tid + i * kScoreThreads;
        if (t < TILE) pre[i] = kbase_ptr[(int64_t)(b + 1) * TILE + t];
      }
    }
    f32x16 acc0 = {}, acc1 = {};
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const uint4 u = tiles[cur][v * kWave + lane];
#pragma unroll
      for (int e = 0; e < OPV; ++e) {
        const Op a = Mfma<T>::from_vec(u, e);
        acc0 = Mfma<T>::mma(a, qop[0][v * OPV + e], acc0);
        acc1 = Mfma<T>::mma(a, qop[1][v * OPV + e], acc1);
      }
    }
    if (has_next) {
#pragma unroll
      for (int i = 0; i < PRE; ++i) {
        const int t = tid + i * kScoreThreads;
        if (t < TILE) tiles[cur ^ 1][t] = pre[i];
      }
    }
    // acc0[r]: query q0 + lane%32, key 8*(r/4) + 4*(lane/32) + r%4 (acc1: query + 32).
    float sa[16], sb[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sa[r] = acc0[r];
      sb[r] = acc1[r];
      half_swap(sa[r], sb[r]);
    }
    // Now, for lane-query q0 + lane: sa[r] -> key 8*(r/4) + r%4, sb[r] -> key 8*(r/4) + 4 + r%4.
    const int kb = b * 32;
    const bool tail = kb + 32 > p.n;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (__ballot(cnt > kCand - 8) != 0) flush();
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float cosv = e < 4 ? sa[4 * g + e] : sb[4 * g + e - 4];
        const int key = kb + 8 * g + e;
        float x = cosv, xc = 0.f;
        if (NOISE) {
          float clean = cosv * p.T;
          if (p.q_len != nullptr) clean *= ql;
          xc = clean;
          const float gv = (valid && key < p.n) ? grow[key] : 0.f;
          x = clean + p.noise_coef * gv;
        }
        bool hit = x > thr;
        if (tail) hit = hit && key < p.n;
        if (hit) {
          cs_[wave][cnt][lane] = x;
          ci_[wave][cnt][lane] = key;
          if (NOISE) cc_[NOISE ? wave : 0][NOISE ? cnt : 0][lane] = xc;
          ++cnt;
        }
      }
    }
    __syncthreads();
  }
  flush();

  if (valid) {
    const int64_t o = ((int64_t)split * p.M + my_q) * p.HC + hc;
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      if (r < p.k) {
        float clean, sel;
        if (NOISE) {
          clean = top.cl[NOISE ? r : 0];
          sel = top.v[r];
        } else {
          clean = top.v[r] * p.T;
          if (p.q_len != nullptr) clean *= ql;
          sel = clean;
        }
        if (p.out_sel != nullptr) p.out_sel[o * p.k + r] = sel;
        p.out_clean[o * p.k + r] = clean;
        p.out_idx[o * p.k + r] = top.id[r];
      }
    }
  }
}

struct Stage2Params {
  const float* part_sel;    // [S, M, HC, k] (null: same as part_clean)
  const float* part_clean;  // [S, M, HC, k]
  const int* part_idx;      // [S, M, HC, k]
  int64_t M;
  int H, n, k, S;
  int32_t* sub_idx;    // [M, HC, k]
  float* sub_scores;   // [M, HC, k]
  int32_t* flat_idx;   // [M, H, k]
  int32_t* slots;      // [M, H, k]
  float* weights;      // [M, H, k]
};

constexpr int kStage2Threads = 64;

// Per-thread LDS columns: [field][entry][thread] keeps the 64 threads of a
// wave on distinct banks for every dynamic access.
template <int KMAX>
__global__ __launch_bounds__(kStage2Threads) void stage2_kernel(Stage2Params p) {
  __shared__ float sel_[2][KMAX][kStage2Threads];
  __shared__ float cl_[2][KMAX][kStage2Threads];
  __shared__ int id_[2][KMAX][kStage2Threads];
  const int t = threadIdx.x;
  const int64_t mh = (int64_t)blockIdx.x * kStage2Threads + t;
  if (mh >= p.M * p.H) return;  // no barriers below
  const int64_t m = mh / p.H;
  const int h = (int)(mh % p.H);
  const int k = p.k;
  const int HC = 2 * p.H;
  const float* psel = p.part_sel != nullptr ? p.part_sel : p.part_clean;

  // Stage-1 result per codebook: merge the split lists (each sorted by
  // select desc, index asc; splits hold disjoint, increasing key ranges).
  for (int c = 0; c < 2; ++c) {
    const int hc = 2 * h + c;
    if (p.S == 1) {
      const int64_t base = (m * HC + hc) * k;
      for (int r = 0; r < k; ++r) {
        sel_[c][r][t] = psel[base + r];
        cl_[c][r][t] = p.part_clean[base + r];
        id_[c][r][t] = p.part_idx[base + r];
      }
    } else {
      int ptr[kMaxSplits];
#pragma unroll
      for (int s = 0; s < kMaxSplits; ++s) ptr[s] = 0;
      for (int r = 0; r < k; ++r) {
        float best = -INFINITY;
        int bid = INT_MAX, bs = 0;
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s) {
          if (s < p.S && ptr[s] < k) {
            const int64_t o = ((s * p.M + m) * HC + hc) * k + ptr[s];
            const float x = psel[o];
            const int xi = p.part_idx[o];
            if (x > best || (x == best && xi < bid)) {
              best = x;
              bid = xi;
              bs = s;
            }
          }
        }
        int pb = 0;
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s) pb = (s == bs) ? ptr[s] : pb;
        const int64_t o = ((bs * p.M + m) * HC + hc) * k + pb;
        sel_[c][r][t] = best;
        cl_[c][r][t] = p.part_clean[o];
        id_[c][r][t] = bid;
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s) ptr[s] += (s == bs) ? 1 : 0;
      }
      const int64_t base = (m * HC + hc) * k;
      for (int r = 0; r < k; ++r) {
        p.sub_idx[base + r] = id_[c][r][t];
        p.sub_scores[base + r] = cl_[c][r][t];
      }
    }
  }

  // Stage 2: frontier walk over rows i (rank in codebook a), ptr[i] = next
  // rank in codebook b.
  int ptr[KMAX];
  float cv[KMAX];
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    ptr[i] = 0;
    cv[i] = i < k ? sel_[0][i][t] + sel_[1][0][t] : -INFINITY;
  }
  float clean[KMAX];
  const int64_t ob = mh * k;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    if (s < k) {
      float best = cv[0];
      int bi = 0, bflat = ptr[0];
#pragma unroll
      for (int i = 1; i < KMAX; ++i) {
        if (i <= s) {
          const int flat = i * k + ptr[i];
          const bool better = cv[i] > best || (cv[i] == best && flat < bflat);
          best = better ? cv[i] : best;
          bi = better ? i : bi;
          bflat = better ? flat : bflat;
        }
      }
      const int rb = min(bflat - bi * k, k - 1);
      clean[s] = cl_[0][bi][t] + cl_[1][rb][t];
      // ids come from keys < n; the clamp only guards non-finite inputs
      // (NaN scores are never inserted) against out-of-range reads later.
      int ia = id_[0][bi][t], ib = id_[1][rb][t];
      ia = (ia >= 0 && ia < p.n) ? ia : 0;
      ib = (ib >= 0 && ib < p.n) ? ib : 0;
      p.slots[ob + s] = ia * p.n + ib;
      p.flat_idx[ob + s] = bflat;
      const float nv = rb + 1 < k ? sel_[0][bi][t] + sel_[1][rb + 1][t] : -INFINITY;
#pragma unroll
      for (int i = 0; i < KMAX; ++i) {
        ptr[i] += (i == bi) ? 1 : 0;
        cv[i] = (i == bi) ? nv : cv[i];
      }
    }
  }
  // Routing softmax over the clean slot scores (memory.py:178).
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < KMAX; ++s)
    if (s < k) mx = fmaxf(mx, clean[s]);
  float sum = 0.f;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    if (s < k) {
      clean[s] = expf(clean[s] - mx);
      sum += clean[s];
    }
  }
#pragma unroll
  for (int s = 0; s < KMAX; ++s)
    if (s < k) p.weights[ob + s] = clean[s] / sum;
}

// ---------------------------------------------------------------- host side
struct Plan {
  int splits, blk_per_split, nblk, kmax;
  int64_t qblocks;
};

static Plan make_plan(int64_t M, int H, int n, int k) {
  Plan pl;
  pl.nblk = (int)cdiv(n, 32);
  pl.qblocks = cdiv(M, kScoreThreads);
  const int64_t base = pl.qblocks * 2 * H;
  int64_t s = cdiv(1024, base);
  s = s < 1 ? 1 : s;
  s = s > kMaxSplits ? kMaxSplits : s;
  s = s > pl.nblk ? pl.nblk : s;
  pl.blk_per_split = (int)cdiv(pl.nblk, s);
  pl.splits = (int)cdiv(pl.nblk, pl.blk_per_split);
  pl.kmax = k <= 16 ? 16 : 32;
  return pl;
}

template <typename T, int HP, bool NOISE, int KMAX>
static void launch_stage1(const ScoreParams& sp, int64_t blocks, hipStream_t s) {
  score_topk_kernel<T, HP, NOISE, KMAX><<<(unsigned)blocks, kScoreThreads, 0, s>>>(sp);
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

static size_t ws_bytes(const Plan& pl, int64_t M, int H, int k, bool noise) {
  const size_t per = (size_t)M * 2 * H * k;
  if (pl.splits == 1) return noise ? per * sizeof(float) : 0;
  return per * pl.splits * (2 * sizeof(float) + sizeof(int));
}

}  // namespace mpl

using namespace mpl;

extern "C" size_t mpl_score_select_workspace_bytes(int64_t M, int H, int n, int half, int k) {
  (void)half;
  if (M <= 0 || H <= 0 || n <= 0 || k <= 0) return 0;
  const Plan pl = make_plan(M, H, n, k);
  return ws_bytes(pl, M, H, k, true);
}

extern "C" int mpl_score_select(const float* q_hat, const float* q_len, const void* packed_keys,
                                int64_t M, int H, int n, int half, int k, int score_dtype,
                                float temperature, const float* gumbel, float noise_coef,
                                void* workspace, size_t workspace_bytes, int32_t* sub_idx,
                                float* sub_scores, int32_t* flat_idx, int32_t* slots,
                                float* weights, void* stream) {
  clear_error();
  MPL_REQUIRE(M >= 0 && H > 0 && n > 0 && half > 0 && k > 0, MPL_EINVAL,
              "mpl_score_select: bad sizes M=%lld H=%d n=%d half=%d k=%d", (long long)M, H, n, half, k);
  MPL_REQUIRE(k <= n && k <= 32, MPL_EUNSUPPORTED, "mpl_score_select: need k <= min(n, 32), got k=%d n=%d",
              k, n);
  MPL_REQUIRE(half <= 128, MPL_EUNSUPPORTED, "mpl_score_select: half=%d > 128", half);
  MPL_REQUIRE((int64_t)n * n < ((int64_t)1 << 31), MPL_EUNSUPPORTED, "mpl_score_select: n*n must be < 2^31");
  MPL_REQUIRE(score_dtype == MPL_F16 || score_dtype == MPL_F32, MPL_EINVAL,
              "mpl_score_select: score_dtype must be MPL_F16 or MPL_F32");
  if (M == 0) return MPL_OK;
  MPL_REQUIRE(q_hat && packed_keys && sub_idx && sub_scores && flat_idx && slots && weights, MPL_EINVAL,
              "mpl_score_select: null buffer");
  const bool noise = gumbel != nullptr;
  const Plan pl = make_plan(M, H, n, k);
  const size_t need = ws_bytes(pl, M, H, k, noise);
  MPL_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr), MPL_EWORKSPACE,
              "mpl_score_select: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  const int HC = 2 * H;
  const size_t per = (size_t)M * HC * k;

  ScoreParams sp;
  sp.q_hat = q_hat;
  sp.q_len = q_len;
  sp.packed = (const uint4*)packed_keys;
  sp.gumbel = gumbel;
  sp.T = temperature;
  sp.noise_coef = noise_coef;
  sp.M = M;
  sp.HC = HC;
  sp.n = n;
  sp.half = half;
  sp.k = k;
  sp.nblk = pl.nblk;
  sp.splits = pl.splits;
  sp.blk_per_split = pl.blk_per_split;
  if (pl.splits == 1) {
    sp.out_sel = noise ? (float*)workspace : nullptr;
    sp.out_clean = sub_scores;
    sp.out_idx = sub_idx;
  } else {
    float* w = (float*)workspace;
    sp.out_sel = w;
    sp.out_clean = w + per * pl.splits;
    sp.out_idx = (int*)(w + 2 * per * pl.splits);
  }
  const int HP = score_dtype == MPL_F16 ? KeyPack<_Float16>::padded_half(half) : KeyPack<float>::padded_half(half);
  const int64_t blocks = pl.qblocks * pl.splits * HC;
  int rc = dispatch_stage1(sp, blocks, score_dtype, HP, noise, pl.kmax, s);
  if (rc) {
    set_error("mpl_score_select: unsupported padded half %d", HP);
    return rc;
  }
  rc = check_launch("mpl_score_select(stage 1)");
  if (rc) return rc;

  Stage2Params p2;
  p2.part_sel = sp.out_sel;
  p2.part_clean = sp.out_clean;
  p2.part_idx = sp.out_idx;
  p2.M = M;
  p2.H = H;
  p2.n = n;
  p2.k = k;
  p2.S = pl.splits;
  p2.sub_idx = sub_idx;
  p2.sub_scores = sub_scores;
  p2.flat_idx = flat_idx;
  p2.slots = slots;
  p2.weights = weights;
  const unsigned g2 = (unsigned)cdiv(M * H, kStage2Threads);
  if (pl.kmax == 16) stage2_kernel<16><<<g2, kStage2Threads, 0, s>>>(p2);
  else stage2_kernel<32><<<g2, kStage2Threads, 0, s>>>(p2);
  return check_launch("mpl_score_select(stage 2)");
}
