// Training-side routing statistics and the load-balance loss of
// memory.py:196-215 on the GPU, on the MFMA tiles of the scoring precision
// (fp16: v_mfma_f32_32x32x16_f16; fp32: v_mfma_f32_32x32x2_f32).
//
//   route_counts_kernel  subkey_counts from the final slots (memory.py:199-204),
//                        the clean stage-1 counts behind f (:206-208) and
//                        slot_counts (:215): integer histograms in LDS,
//                        flushed with float atomics of whole numbers
//   balance_fwd_kernel   per (token m, codebook hc), over all n sub-keys, the
//                        log-sum-exp of the balance logits z_n = T_eff cos_n
//                        and r_m = sum_n f_n softmax(z)_n, online in one sweep
//                        of MFMA score tiles; balance = n/(2H M) sum r
//                        (memory.py:210-213)
//   revive_kernel        revive_dead_keys (memory.py:243-281) in place
//   balance_grad_kernel  the gradient of balance (dense over n) with respect
//                        to the normalised queries and sub-keys, as two MFMA
//                        passes that recompute the score tiles; the sub-key
//                        pass also takes the routed term (d sub_scores of the
//                        selected keys), so the whole d k_hat is one dense
//                        pass; the same kernel computes key_diversity_loss
//                        (memory.py:230-240) and its gradient from the Gram
//                        tiles of the sub-keys
//
// With f fixed (stop_gradient, memory.py:208) the loss is
// n/(2H M) sum_{m,hc} r_m, so the gradient with respect to the logits is
//   dz_mn = c p_mn (f_n - r_m),   c = g n / (2H M),
// and with T_eff = T rho_m (rho_m = q_len_m when the balance logits are the
// query-scaled scores, memory.py:210 with balance_temperature_grad, else 1)
//   d q_hat_m = T rho_m sum_n dz_mn k_hat_n
//   d k_hat_n = T sum_m dz_mn rho_m q_hat_m.
// The MFMA operand p (f - r) is scaled per codebook by
// sigma = 2^floor(log2(n/4)) / max_n f_n: |p (f - r)| <= max f, so the scaled
// operand stays below n/4 while its typical size (about 1/n^2 unscaled) no
// longer underflows fp16.
#include <math.h>

#include "common.h"
#include "layout.h"
#include "mfma.h"

namespace mpl {
namespace {

constexpr int kBalThreads = 256;  // four waves
constexpr int kBalWaves = kBalThreads / kWave;
constexpr int kRowsPerGroup = 32 * kBalWaves;  // fixed-side rows per workgroup
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kRtPitch = 36;  // floats per key row of the routed-term tile (32 queries + bank padding)

// Operand shapes of one scoring precision E (_Float16: v_mfma_f32_32x32x16_f16,
// float: v_mfma_f32_32x32x2_f32) as the balance kernels use them:
//   NCH  MFMAs per 32-row block (K = half padded to HP);
//   NV   16-byte vectors per lane per block of a normal pack (layout.h);
//   OPV  MFMA operands per 16-byte vector;
//   RPO  score-tile registers that form one contraction operand (the tile
//        rows of register r are 8(r/4) + 4(l/32) + r%4), and NOP = 16 / RPO
//        contraction MFMAs per 32-dim block of the output;
//   TVPD 16-byte vectors per lane per 32-dim block of a transposed pack.
template <typename E>
struct BalOps;

template <>
struct BalOps<_Float16> {
  typedef Mfma<_Float16> MF;
  typedef KeyPack<_Float16> KP;
  static constexpr int kRowsPerOp = 8;
  static constexpr int kElemsPerVec = 8;
  __device__ static half8 from_rows(const float* g) {
    half8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (_Float16)g[j];
    return h;
  }
};

template <>
struct BalOps<float> {
  typedef Mfma<float> MF;
  typedef KeyPack<float> KP;
  static constexpr int kRowsPerOp = 1;
  static constexpr int kElemsPerVec = 4;
  __device__ static float from_rows(const float* g) { return g[0]; }
};

template <typename E, int HP>
struct BalShape {
  typedef BalOps<E> Ops;
  static constexpr int NCH = HP / Ops::KP::kChunk;
  static constexpr int NV = Ops::KP::vectors_per_lane(HP);
  static constexpr int OPV = Ops::KP::kOpsPerVec;
  static constexpr int RPO = Ops::kRowsPerOp;
  static constexpr int NOP = 16 / RPO;
  static constexpr int TVPD = 16 / Ops::kElemsPerVec;
  static constexpr int ND = (HP + 31) / 32;
  static_assert(NCH == NV * OPV, "a normal pack holds every MFMA operand of a block");
  static_assert(NOP == TVPD * OPV, "a transposed pack holds every contraction operand of a block");
};

// ------------------------------------------------------------- counting
__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ x, int64_t n) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) x[i] = 0.f;
}

__global__ __launch_bounds__(64) void fill_value_kernel(float* __restrict__ x, int64_t n, float v) {
  for (int64_t i = blockIdx.x * 64 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 64) x[i] = v;
}

// Three buffers cleared by one launch (null ones skipped): the count
// outputs, which every launch of the count kernel needs at zero.
__global__ __launch_bounds__(256) void fill_zero3_kernel(float* __restrict__ a, int64_t na, float* __restrict__ b,
                                                         int64_t nb, float* __restrict__ c, int64_t nc) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < na + nb + nc; i += stride) {
    if (i < na) a[i] = 0.f;
    else if (i < na + nb) b[i - na] = 0.f;
    else c[i - na - nb] = 0.f;
  }
}

// Workgroup b covers head h = b % H and tokens [t0, t0 + tpg).  With use_lds
// the two sub-key histograms and the two clean histograms of head h ([4][n]
// ints) are built in LDS and added to the outputs once per workgroup.  Ids
// outside their range are not counted.  P2: k and n are powers of two
// (kshift = log2 k, nshift = log2 n), so the id positions and the slot's
// sub-key pair come from shifts and masks rather than integer divisions.
template <bool P2>
__global__ __launch_bounds__(256) void route_counts_kernel(const int32_t* __restrict__ slots,
                                                           const int32_t* __restrict__ clean, int64_t M, int H,
                                                           int n, int k, int kshift, int nshift, int64_t tpg,
                                                           int use_lds, float* __restrict__ sub_counts,
                                                           float* __restrict__ clean_counts,
                                                           float* __restrict__ slot_counts) {
  extern __shared__ int hist[];
  const int tid = threadIdx.x;
  const int h = blockIdx.x % H;
  const int64_t t0 = (int64_t)(blockIdx.x / H) * tpg;
  const int64_t t1 = t0 + tpg < M ? t0 + tpg : M;
  const int64_t N = (int64_t)n * n;
  const bool do_sub = sub_counts != nullptr;
  const bool do_clean = clean_counts != nullptr && clean != nullptr;
  if (use_lds) {
    for (int i = tid; i < 4 * n; i += 256) hist[i] = 0;
    __syncthreads();
  }
  if (t1 > t0) {
    // ids of token m, head h: slots[(m H + h) k + j], clean[(m H + h) 2k + c k + j]
    const int ne = (int)(t1 - t0) * k;
    const int32_t* sbase = slots + (t0 * H + h) * k;
    for (int e = tid; e < ne; e += 256) {
      const int mm = P2 ? e >> kshift : e / k;
      const int j = e - mm * k;
      const int s = sbase[(int64_t)mm * H * k + j];
      if (s < 0 || s >= N) continue;
      if (slot_counts != nullptr) unsafeAtomicAdd(&slot_counts[s], 1.0f);
      if (do_sub) {
        const int a = P2 ? s >> nshift : s / n;
        const int b2 = s - a * n;
        if (use_lds) {
          atomicAdd(&hist[a], 1);
          atomicAdd(&hist[n + b2], 1);
        } else {
          unsafeAtomicAdd(&sub_counts[(2 * h) * n + a], 1.0f);
          unsafeAtomicAdd(&sub_counts[(2 * h + 1) * n + b2], 1.0f);
        }
      }
    }
    if (do_clean) {
      const int nc = (int)(t1 - t0) * 2 * k;
      const int32_t* cbase = clean + (t0 * H + h) * 2 * k;
      for (int e = tid; e < nc; e += 256) {
        const int mm = P2 ? e >> (kshift + 1) : e / (2 * k);
        const int r = e - mm * 2 * k;  // c * k + j
        const int c = P2 ? r >> kshift : r / k;
        const int i = cbase[(int64_t)mm * H * 2 * k + r];
        if (i < 0 || i >= n) continue;
        if (use_lds)
          atomicAdd(&hist[(2 + c) * n + i], 1);
        else
          unsafeAtomicAdd(&clean_counts[(2 * h + c) * n + i], 1.0f);
      }
    }
  }
  if (use_lds) {
    __syncthreads();
    for (int i = tid; i < 4 * n; i += 256) {
      const int v = hist[i];
      const int which = P2 ? i >> nshift : i / n, key = i - which * n;
      float* dst = which < 2 ? sub_counts : (do_clean ? clean_counts : nullptr);
      if (v == 0 || dst == nullptr) continue;
      unsafeAtomicAdd(&dst[(2 * h + (which & 1)) * n + key], (float)v);
    }
  }
}

// ------------------------------------------------------------- forward
struct BalFwdParams {
  const float* q;         // raw queries [M, HC, half]
  const uint4* packed;    // packed sub-keys (layout.h, the kernel's precision)
  const float* counts;    // clean counts [HC, n]
  float inv_mk;           // 1 / (M k)
  const float* T;         // device scalar: the clamped temperature
  int scaled;             // T_eff = T * q_len
  int64_t M;
  int HC, n, half, nblk;
  float4* state;          // [HC, M]: (log2-sum-exp2 of z log2e, r, T_eff log2e, 0)
  float* parts;           // [grid]: sum of r over the workgroup's queries
};

// One block of 32 keys staged in LDS by the whole workgroup, plain loads
// through registers, double buffered: iteration j computes on buffer j%2
// while block j+1 waits in registers.
template <int TILE>
struct Stage {
  static constexpr int kPer = (TILE + kBalThreads - 1) / kBalThreads;
  uint4 r[kPer];
  __device__ __forceinline__ void load(const uint4* src, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = tid + i * kBalThreads;
      r[i] = idx < TILE ? src[idx] : uint4{0, 0, 0, 0};
    }
  }
  __device__ __forceinline__ void store(uint4* dst, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = tid + i * kBalThreads;
      if (idx < TILE) dst[idx] = r[i];
    }
  }
};

// Sum over the 256 threads of a workgroup in a fixed order (every thread
// must call it; the result is returned to all).
__device__ __forceinline__ float block_sum256(float v, float* sh) {
  sh[threadIdx.x] = v;
  __syncthreads();
  for (int off = 128; off >= 1; off >>= 1) {
    if ((int)threadIdx.x < off) sh[threadIdx.x] += sh[threadIdx.x + off];
    __syncthreads();
  }
  const float r = sh[0];
  __syncthreads();
  return r;
}

// Lanes l and l+32 hold the same query; returns the partner lane's value.
__device__ __forceinline__ float partner(float v, int par) {
  float a = v, b = v;
  half_swap(a, b);
  return par ? a : b;
}

template <typename E, int HP>
__global__ __launch_bounds__(kBalThreads) void balance_fwd_kernel(BalFwdParams p) {
  typedef BalShape<E, HP> Sh;
  typedef typename Sh::Ops::MF MF;
  constexpr int NCH = Sh::NCH, OPV = Sh::OPV;
  constexpr int TILE = Sh::NV * kWave;
  __shared__ uint4 tiles[2][TILE];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, par = lane >> 5;
  const int hc = blockIdx.x % p.HC;
  const int64_t my_q = (int64_t)(blockIdx.x / p.HC) * kRowsPerGroup + wave * 32 + (lane & 31);
  const bool valid = my_q < p.M;

  // the raw query, normalised (memory.py:30-31, 136-137)
  const float* qrow = p.q + (valid ? (my_q * p.HC + hc) * (int64_t)p.half : 0);
  float x[NCH][MF::kQElems];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) MF::load_q_raw(qrow, valid, p.half, c, lane, x[c], ss);
  const float tot = ss + partner(ss, par) + 1e-6f;
  const float rn = 1.0f / sqrtf(tot);
  typename MF::Op qop[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) qop[c] = MF::scale_q(x[c], rn);
  const float rho = p.scaled ? sqrtf(tot) / sqrtf((float)p.half) : 1.f;
  const float t2 = *p.T * rho * kLog2e;

  const float* cnt = p.counts + (int64_t)hc * p.n;
  const uint4* kb = p.packed + (int64_t)hc * p.nblk * TILE;
  Stage<TILE> st;
  st.load(kb, tid);
  st.store(tiles[0], tid);
  __syncthreads();
  // online base-2 log-sum-exp over this lane's keys: z2 <= mx, S = sum 2^(z2-mx), F = sum cnt 2^(z2-mx)
  float mx = -INFINITY, S = 0.f, F = 0.f;
  for (int blk = 0; blk < p.nblk; ++blk) {
    const int cur = blk & 1;
    if (blk + 1 < p.nblk) st.load(kb + (int64_t)(blk + 1) * TILE, tid);
    f32x16 acc = f32x16{};
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      acc = MF::mma(MF::from_vec(tiles[cur][(c / OPV) * kWave + lane], c % OPV), qop[c], acc);
    float z[16], fv[16];
    float bm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = blk * 32 + 8 * (r >> 2) + 4 * par + (r & 3);
      fv[r] = cnt[key < p.n ? key : p.n - 1];
      z[r] = key < p.n ? acc[r] * t2 : -INFINITY;
      bm = fmaxf(bm, z[r]);
    }
    if (bm > mx) {
      const float sc = exp2f(mx - bm);  // 0 while mx is -inf
      S *= sc;
      F *= sc;
      mx = bm;
    }
    const float mu = mx == -INFINITY ? 0.f : mx;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = exp2f(z[r] - mu);
      S += e;
      F = fmaf(fv[r], e, F);
    }
    if (blk + 1 < p.nblk) st.store(tiles[cur ^ 1], tid);
    __syncthreads();
  }
  const float mo = partner(mx, par), So = partner(S, par), Fo = partner(F, par);
  const float mm = fmaxf(mx, mo);
  const float s1 = mx == -INFINITY ? 0.f : exp2f(mx - mm);
  const float s2 = mo == -INFINITY ? 0.f : exp2f(mo - mm);
  const float St = S * s1 + So * s2, Ft = F * s1 + Fo * s2;
  const float r = Ft / St * p.inv_mk;
  if (valid && par == 0) p.state[(int64_t)hc * p.M + my_q] = make_float4(mm + log2f(St), r, t2, 0.f);
  __shared__ float red[kBalThreads];
  const float wsum = block_sum256((valid && par == 0) ? r : 0.f, red);
  if (tid == 0) p.parts[blockIdx.x] = wsum;
}

// balance = coef * sum of the workgroups' sums of r, fixed order.
__global__ __launch_bounds__(1024) void balance_loss_kernel(const float* __restrict__ parts, int64_t count,
                                                            float coef, float* __restrict__ loss) {
  __shared__ double part[1024];
  const int tid = threadIdx.x;
  double s = 0.0;
  for (int64_t i = tid; i < count; i += 1024) s += (double)parts[i];
  part[tid] = s;
  __syncthreads();
  for (int off = 512; off >= 1; off >>= 1) {
    if (tid < off) part[tid] += part[tid + off];
    __syncthreads();
  }
  if (tid == 0) *loss = (float)(part[0] * (double)coef);
}

// ------------------------------------------------------------- backward
// Operand packs of fp32 rows X(hc, row, d) = X[hc*s_hc + row*s_row + d]
// (rows >= nrows and dims >= half are zero), optionally times scale(hc, row),
// converted to the precision E:
//   normal      out[hc][blk][v][lane]: lane l holds row 32 blk + l%32, dims
//               KeyPack<E>::dim_of(v, i, l) (the scoring operand, as the
//               sub-key pack of layout.h);
//   transposed  out[hc][blk][db][w][lane]: element i of vector w holds dim
//               32 db + l%32 of row 32 blk + 8(r/4) + 4(l/32) + r%4 with
//               r = w * (elements per vector) + i: the A operand that meets
//               the score tile's registers as the B operand (fp16: registers
//               8w..8w+7 in one MFMA; fp32: register r in MFMA r).
template <bool TRANS, typename E, int HP>
__global__ __launch_bounds__(256) void pack_rows_kernel(const float* __restrict__ X, int64_t s_hc, int64_t s_row,
                                                        int64_t nrows, int HC, int half,
                                                        const float* __restrict__ scale, int64_t sc_hc,
                                                        int64_t sc_row, int64_t nblk, uint4* __restrict__ out) {
  typedef BalShape<E, HP> Sh;
  typedef typename Sh::Ops::KP KP;
  constexpr int EPV = Sh::Ops::kElemsPerVec;
  constexpr int PER_BLK = TRANS ? Sh::ND * Sh::TVPD : Sh::NV;  // 16-byte vectors per lane per block
  const int64_t total = (int64_t)HC * nblk * PER_BLK * kWave;
  for (int64_t t = blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
    const int lane = (int)(t % kWave);
    const int64_t u = t / kWave;
    const int w = (int)(u % PER_BLK);
    const int64_t blk = (u / PER_BLK) % nblk;
    const int hc = (int)(u / PER_BLK / nblk);
    const float* base = X + (int64_t)hc * s_hc;
    float e[EPV];
    if (!TRANS) {
      const int64_t row = blk * 32 + (lane & 31);
      const float sc = (row < nrows && scale != nullptr) ? scale[hc * sc_hc + row * sc_row] : 1.f;
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        const int d = KP::dim_of(w, i, lane);
        e[i] = (row < nrows && d < half) ? base[row * s_row + d] * sc : 0.f;
      }
    } else {
      const int wv = w % Sh::TVPD, db = w / Sh::TVPD;
      const int d = 32 * db + (lane & 31);
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        const int r = wv * EPV + i;
        const int64_t row = blk * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const bool ok = row < nrows && d < half;
        const float sc = (ok && scale != nullptr) ? scale[hc * sc_hc + row * sc_row] : 1.f;
        e[i] = ok ? base[row * s_row + d] * sc : 0.f;
      }
    }
    out[t] = KP::pack(e);
  }
}

// Both fp16 packs of unscaled rows with half == HP (pack_rows_kernel<false>
// and <true> of the same rows) from one read of them: workgroup (hc, blk)
// stages the block's 32 rows x HP fp32 dims in LDS with 16-byte loads, then
// writes the normal pack (a vector is 8 consecutive dims of one row) and the
// transposed pack (a vector is one dim of 8 rows) from the tile.  The same
// fp16 values in the same places as the two separate launches.
// NORM: X holds raw rows, normalised here exactly as l2norm_kernel does
// (16 partial sums of squares per row, j = l, l + 16, ... by fma from 0,
// joined in its xor-butterfly order, then x * (1 / sqrt(sum + eps))), so the
// packs equal those of the normalised rows bit for bit.
template <int HP, bool NORM>
__global__ __launch_bounds__(256) void pack_rows_both_f16_kernel(const float* __restrict__ X, int64_t s_hc,
                                                                 int64_t s_row, int64_t nrows, int64_t nblk,
                                                                 float eps, uint4* __restrict__ out_n,
                                                                 uint4* __restrict__ out_t) {
  constexpr int PITCH = HP + 4;  // floats per staged row (16-byte aligned rows, shifted banks)
  constexpr int V4 = HP / 4;     // 16-byte vectors per row
  constexpr int NV = HP / 16;    // normal pack: vectors per lane per block
  constexpr int NT = HP / 16;    // transposed pack: HP / 32 dim groups x 2 vectors
  __shared__ float tile[32 * PITCH];
  __shared__ float psum[NORM ? 32 : 1][NORM ? 17 : 1];
  const int64_t blk = blockIdx.x % nblk;
  const int64_t hc = blockIdx.x / nblk;
  const float* base = X + hc * s_hc;
  for (int t = threadIdx.x; t < 32 * V4; t += 256) {
    const int rr = t / V4, c4 = t % V4;
    const int64_t row = blk * 32 + rr;
    const float4 v = row < nrows ? *(const float4*)(base + row * s_row + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
    *(float4*)(tile + rr * PITCH + 4 * c4) = v;
  }
  __syncthreads();
  if constexpr (NORM) {
    for (int t = threadIdx.x; t < 32 * 16; t += 256) {
      const int rr = t >> 4, l = t & 15;
      float sq = 0.f;
      for (int j = l; j < HP; j += 16) sq = fmaf(tile[rr * PITCH + j], tile[rr * PITCH + j], sq);
      psum[NORM ? rr : 0][NORM ? l : 0] = sq;
    }
    __syncthreads();
    if (threadIdx.x < 32) {
      const float* ps = psum[NORM ? threadIdx.x : 0];
      float t8[8], t4[4];
#pragma unroll
      for (int l = 0; l < 8; ++l) t8[l] = ps[l] + ps[l + 8];
#pragma unroll
      for (int l = 0; l < 4; ++l) t4[l] = t8[l] + t8[l + 4];
      const float v0 = t4[0] + t4[2], v1 = t4[1] + t4[3];
      const float tot = (v0 + v1) + eps;
      psum[NORM ? threadIdx.x : 0][NORM ? 16 : 0] = 1.0f / sqrtf(tot);
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 32 * HP; t += 256) {
      const int rr = t / HP, j = t % HP;
      tile[rr * PITCH + j] = tile[rr * PITCH + j] * psum[NORM ? rr : 0][NORM ? 16 : 0];
    }
    __syncthreads();
  }
  const int64_t ob = (hc * nblk + blk) * (int64_t)(NV * kWave);
  for (int t = threadIdx.x; t < NV * kWave; t += 256) {
    const int v = t / kWave, l = t % kWave;
    const float* src = tile + (l & 31) * PITCH + 16 * v + 8 * (l >> 5);
    const float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
    const float e[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    half8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16)e[i];
    out_n[ob + t] = __builtin_bit_cast(uint4, h);
  }
  for (int t = threadIdx.x; t < NT * kWave; t += 256) {
    const int w = t / kWave, l = t % kWave;
    const int wv = w & 1, d = 32 * (w >> 1) + (l & 31);
    half8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = wv * 8 + i;
      h[i] = (_Float16)tile[(8 * (r >> 2) + 4 * (l >> 5) + (r & 3)) * PITCH + d];
    }
    out_t[ob + t] = __builtin_bit_cast(uint4, h);
  }
}

// Per codebook maxima of |d_sub| and q_len over a range of tokens: workgroup
// b covers tokens [b * tpg, (b + 1) * tpg) and writes part[b][hc] =
// (max |d_sub|, max q_len).  Maxima do not depend on the order of the
// comparisons, so the result is deterministic.
__global__ __launch_bounds__(256) void bwd_max_kernel(const float* __restrict__ d_sub,
                                                      const float* __restrict__ q_len, int64_t M, int HC, int k,
                                                      int64_t tpg, float2* __restrict__ part) {
  __shared__ float red[2][256];
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)blockIdx.x * tpg;
  const int64_t t1 = t0 + tpg < M ? t0 + tpg : M;
  for (int hc = 0; hc < HC; ++hc) {
    float dm = 0.f, qm = 0.f;
    if (d_sub != nullptr)
      for (int64_t e = t0 * k + tid; e < t1 * k; e += 256) {
        const int64_t m = e / k;
        dm = fmaxf(dm, fabsf(d_sub[(m * HC + hc) * k + (e - m * k)]));
      }
    if (q_len != nullptr)
      for (int64_t m = t0 + tid; m < t1; m += 256) qm = fmaxf(qm, q_len[m * HC + hc]);
    red[0][tid] = dm;
    red[1][tid] = qm;
    __syncthreads();
    for (int off = 128; off >= 1; off >>= 1) {
      if (tid < off) {
        red[0][tid] = fmaxf(red[0][tid], red[0][tid + off]);
        red[1][tid] = fmaxf(red[1][tid], red[1][tid + off]);
      }
      __syncthreads();
    }
    if (tid == 0) part[(int64_t)blockIdx.x * HC + hc] = make_float2(red[0][0], red[1][0]);
    __syncthreads();
  }
}

// bwd_max_kernel in one coalesced pass, when a token's HC * k entries of
// d_sub are V = HC * k / 4 16-byte vectors and V and HC divide 256: thread
// t reads vector t % V of every (256 / V)-th token, which always lies in
// codebook (t % V) / (k / 4); the threads of a codebook then meet in LDS.
// The same maxima as bwd_max_kernel (a maximum does not depend on order).
__global__ __launch_bounds__(256) void bwd_max_vec_kernel(const float* __restrict__ d_sub,
                                                          const float* __restrict__ q_len, int64_t M, int HC, int k,
                                                          int64_t tpg, float2* __restrict__ part) {
  __shared__ float red[2][256];
  const int tid = threadIdx.x;
  const int V = HC * k / 4;
  const int64_t t0 = (int64_t)blockIdx.x * tpg;
  const int64_t t1 = t0 + tpg < M ? t0 + tpg : M;
  float dm = 0.f, qm = 0.f;
  if (d_sub != nullptr) {
    const float4* d4 = (const float4*)d_sub;
    for (int64_t m = t0 + tid / V; m < t1; m += 256 / V) {
      const float4 v = d4[m * V + tid % V];
      dm = fmaxf(dm, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
  }
  if (q_len != nullptr)
    for (int64_t m = t0 + tid / HC; m < t1; m += 256 / HC) qm = fmaxf(qm, q_len[m * HC + tid % HC]);
  red[0][tid] = dm;
  red[1][tid] = qm;
  __syncthreads();
  if (tid < HC) {
    float a = 0.f, b = 0.f;
    for (int j = tid * (k / 4); j < 256; j += V)  // vectors of codebook tid: (j % V) / (k / 4) == tid
      for (int i = 0; i < k / 4; ++i) a = fmaxf(a, red[0][j + i]);
    for (int j = tid; j < 256; j += HC) b = fmaxf(b, red[1][j]);
    part[(int64_t)blockIdx.x * HC + tid] = make_float2(a, b);
  }
}

// Per codebook: sigma = 2^floor(log2(n/4)) / max f (the d q_hat operand
// scale, f = counts / (M k)) and S = (bound on |d cos| of the sub-key pass) /
// 2^14, the bound being T (max q_len if query_scale) max |d_sub| plus the
// balance term's T (max q_len if its logits carry it) |c| max f.  One
// workgroup per codebook over the partial maxima.
__global__ __launch_bounds__(256) void bwd_scale_kernel(const float* __restrict__ counts,
                                                        const float2* __restrict__ part, int nparts, int n,
                                                        int HC, float inv_mk, const float* __restrict__ g, float coef,
                                                        const float* __restrict__ Tp, int btg, int qs,
                                                        float* __restrict__ sigma, float* __restrict__ S) {
  __shared__ float red[3][256];
  const int hc = blockIdx.x, tid = threadIdx.x;
  float fm = 0.f, dm = 0.f, qm = 0.f;
  if (counts != nullptr)
    for (int i = tid; i < n; i += 256) fm = fmaxf(fm, counts[(int64_t)hc * n + i]);
  for (int b = tid; b < nparts; b += 256) {
    const float2 v = part[(int64_t)b * HC + hc];
    dm = fmaxf(dm, v.x);
    qm = fmaxf(qm, v.y);
  }
  red[0][tid] = fm;
  red[1][tid] = dm;
  red[2][tid] = qm;
  __syncthreads();
  for (int off = 128; off >= 1; off >>= 1) {
    if (tid < off)
      for (int j = 0; j < 3; ++j) red[j][tid] = fmaxf(red[j][tid], red[j][tid + off]);
    __syncthreads();
  }
  if (tid == 0) {
    const float fmax = red[0][0] * inv_mk;
    if (sigma != nullptr) {
      const float p2 = exp2f(floorf(log2f(fmaxf((float)n * 0.25f, 1.f))));
      sigma[hc] = fmax > 0.f ? p2 / fmax : 1.f;
    }
    const float T = *Tp;
    const float rho_r = qs ? red[2][0] : 1.f;
    const float rho_b = (btg && qs) ? red[2][0] : 1.f;
    float bound = T * rho_r * red[1][0];
    if (g != nullptr) bound += T * rho_b * fabsf(*g * coef) * fmax;
    const float sc = bound * (1.0f / 16384.f);
    S[hc] = (sc > 0.f && sc < INFINITY) ? sc : 1.f;
  }
}

struct BalGradParams {
  const uint4* fix;     // fixed side, normal pack [HC][fblk][NV][64]
  const uint4* str;     // streamed side, normal pack [HC][sblk][NV][64]
  const uint4* strT;    // streamed side, transposed pack [HC][sblk][ND][TVPD][64]
  const float4* state;  // [HC, M] from the forward
  const float* counts;  // clean counts [HC, n]
  const float* sigma;   // [HC]
  const float* g;       // d loss / d balance (device scalar)
  float inv_mk, coef;   // 1 / (M k), n / (HC M)
  const float* T;       // device scalar: the clamped temperature (DQ / DK; null for Div)
  int64_t M;
  int HC, n, half;
  int64_t fblk, sblk;  // blocks of 32 rows on the fixed / streamed side
  int splits;
  int64_t sblk_per_split;
  const float* rho;  // DQ: [M, HC] output scale (q_len in the balance logits) or null
  float* out;        // DQ: d q_hat [M, HC, half]; DK: partial d k_hat [splits, HC, n, half]
  float* u;          // DQ: [HC, M] c sum_n p (f - r) cos, or null; Div: per-workgroup sums of squares
  // kModeDK and kModeDQR
  int bal;                // balance terms on (g, state, counts valid)
  const int32_t* sub_idx; // routed term: stage-1 ids [M, HC, k], or null
  const float* d_sub;     // routed term: d sub_scores [M, HC, k]
  const float* qlen_rt;   // routed term: q_len [M, HC] with query_scale, or null
  int k;
  const float* dk_scale;  // [HC] operand scale S: the operand is dcos / S, d k_hat = S * acc
  // kModeDQR only
  const float* q_raw;     // raw queries [M, HC, half]
  float eps;              // the l2 normalisation's epsilon
  float* dq;              // d queries [M, HC, half] (through the normalisation)
};

enum { kModeDQ = 0, kModeDK = 1, kModeDiv = 2, kModeDQR = 3 };

// kModeDQ: the fixed side is 32 queries per wave (B operand), sub-key blocks
// stream.  kModeDK: the fixed side is 32 sub-keys per wave, blocks of 32
// queries stream (the query range is split over `splits` workgroups); the
// operand is the whole d cos of the sub-keys (balance term and, with
// sub_idx, the routed term d_sub * T (* q_len) of memory.py:150-163) over S.
// The routed entries of each query block whose ids fall in the workgroup's
// 128 sub-keys are scattered into an LDS tile [key][query] one block ahead;
// every lane reads its 16 entries and zeroes them, so the tile is clean when
// its buffer comes round again.
// kModeDQR: kModeDQ with the routed term of the queries (d_sub * T of
// memory.py:150-163 at the k selected sub-keys of each query) in the same
// operand, over the same scale S as kModeDK (the bound of both terms), the
// routed entries of the workgroup's 128 queries held in registers and
// scattered into an LDS tile [query][key] one key block ahead; the epilogue
// takes d q_hat through the l2 normalisation backward to d queries (no
// query_scale, no balance temperature gradient).
// kModeDiv: both sides are the sub-keys of one codebook (the Gram matrix of
// key_diversity_loss); the operand is the off-diagonal cosine itself and each
// lane also sums its squares into u[workgroup * 256 + thread].
// Each streamed block: score tile C (rows = streamed, columns = fixed), the
// operand g in the kernel's precision, and for every 32-dim block db of the
// output acc[db] += strT[db] . g (fp16: two MFMAs, K = 16 rows each; fp32:
// sixteen, K = 2 rows each).
template <int MODE, typename E, int HP>
__global__ __launch_bounds__(kBalThreads) void balance_grad_kernel(BalGradParams p) {
  typedef BalShape<E, HP> Sh;
  typedef typename Sh::Ops Ops;
  typedef typename Ops::MF MF;
  constexpr bool DK = MODE == kModeDK || MODE == kModeDiv;  // the fixed side is sub-keys
  constexpr bool DIV = MODE == kModeDiv;
  constexpr bool DQR = MODE == kModeDQR;
  constexpr bool RT = MODE == kModeDK || DQR;  // an LDS tile of routed entries [fixed row][streamed row]
  const float Tv = DIV ? 0.f : *p.T;  // Div mode has no temperature (p.T null)
  constexpr int NCH = Sh::NCH, OPV = Sh::OPV, ND = Sh::ND;
  constexpr int TN = Sh::NV * kWave, TT = ND * Sh::TVPD * kWave, TILE = TN + TT;
  __shared__ uint4 tiles[2][TILE];
  __shared__ __attribute__((aligned(16)))
  float rtile[RT ? 2 : 1][RT ? kRowsPerGroup : 1][RT ? kRtPitch : 1];
  // kModeDK: the forward state of the streamed block's 32 queries; kModeDQ
  // and kModeDQR: the clean counts of its 32 sub-keys (in .x); staged with
  // the block's tiles (one block ahead, double-buffered) so that the
  // per-element reads come from LDS instead of global memory
  __shared__ float4 sstate[MODE != kModeDiv ? 2 : 1][MODE != kModeDiv ? 32 : 1];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, par = lane >> 5;
  const int hc = blockIdx.x % p.HC;
  const int64_t rest = blockIdx.x / p.HC;
  const int split = (int)(rest % p.splits);
  const int64_t fg = rest / p.splits;
  const bool route = RT && p.sub_idx != nullptr;
  const bool bal = MODE != kModeDK || p.bal != 0;
  const int64_t fb = fg * kBalWaves + wave;  // this wave's fixed block
  const int64_t nfix = DK ? p.n : p.M;
  const int64_t nstr = (DK && !DIV) ? p.M : p.n;
  const bool grad = p.out != nullptr;  // kModeDiv may ask for the loss only
  const int64_t my_f = fb * 32 + (lane & 31);
  const bool valid = my_f < nfix;
  const int64_t fbc = fb < p.fblk ? fb : p.fblk - 1;

  typename MF::Op fop[NCH];
  {
    const uint4* src = p.fix + ((int64_t)hc * p.fblk + fbc) * TN;
#pragma unroll
    for (int c = 0; c < NCH; ++c) fop[c] = MF::from_vec(src[(c / OPV) * kWave + lane], c % OPV);
  }
  const float sig = (MODE == kModeDQ) ? p.sigma[hc] : 1.f;
  const float fs = p.inv_mk * sig;  // scaled f per count
  const float* cnt = bal && !DIV ? p.counts + (int64_t)hc * p.n : nullptr;
  const float4* sth = bal && !DIV ? p.state + (int64_t)hc * p.M : nullptr;
  const float cc = (bal && !DIV) ? *p.g * p.coef : 1.f;
  const float invS = RT ? 1.f / p.dk_scale[hc] : 1.f;
  const float a1 = cc * Tv * invS;  // kModeDQR: the balance term's factor on the operand
  // per-lane constants of the fixed row
  float4 fst = make_float4(0.f, 0.f, 0.f, 0.f);
  float ffix = 0.f;
  if (MODE == kModeDK && bal)
    ffix = cnt[valid ? my_f : 0] * p.inv_mk;
  else if (MODE == kModeDQ || DQR)
    fst = sth[valid ? my_f : 0];
  const float rs_fix = fst.y * sig;
  const int64_t k0 = fg * kRowsPerGroup;  // kModeDK: the workgroup's first sub-key
  const int f_loc = wave * 32 + (lane & 31);
  // kModeDK: routed entries of query block b whose ids are in [k0, k0 + 128)
  // go to rtile[x][id - k0][query - 32 b] (ids of one query are distinct).
  // rload fetches this thread's (at most 4: k <= 32) entries of block b into
  // registers, rstore writes them; the loads of block b+1 are issued with the
  // tile loads and written after the block's MFMAs.
  constexpr int kRtPer = (32 * 32 + kBalThreads - 1) / kBalThreads;
  int rrel[kRtPer], rq[kRtPer];
  float rval[kRtPer];
  auto rload = [&](int64_t b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kRtPer; ++i) {
      const int e = tid + i * kBalThreads;
      rrel[i] = -1;
      if (MODE != kModeDK || e >= 32 * p.k) continue;
      const int qlo = e / p.k, j = e - qlo * p.k;
      const int64_t m = b * 32 + qlo;
      if (m >= p.M) continue;
      const int64_t o = (m * p.HC + hc) * p.k + j;
      const int64_t rel = (int64_t)p.sub_idx[o] - k0;
      if (rel < 0 || rel >= kRowsPerGroup) continue;
      const float sc = p.qlen_rt != nullptr ? p.qlen_rt[m * p.HC + hc] : 1.f;
      rrel[i] = (int)rel;
      rq[i] = qlo;
      rval[i] = p.d_sub[o] * sc * Tv;
    }
  };
  auto rstore = [&](int x) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kRtPer; ++i)
      if (MODE == kModeDK && rrel[i] >= 0) rtile[RT ? x : 0][RT ? rrel[i] : 0][RT ? rq[i] : 0] = rval[i];
  };
  // kModeDQR: entry e = tid + 256 i of the workgroup's 128 queries x k
  // (k <= 16: at most 8 per thread), id and d_sub T / S, loaded once;
  // qstore writes those of key block b to rtile[x][query][id - 32 b]
  constexpr int kRtQ = DQR ? 8 : 1;
  int qid[kRtQ], qrow[kRtQ];
  float qval[kRtQ];
  if constexpr (DQR) {
#pragma unroll
    for (int i = 0; i < kRtQ; ++i) {
      const int e = tid + i * kBalThreads;
      qid[i] = -1;
      qrow[i] = 0;
      qval[i] = 0.f;
      if (e >= kRowsPerGroup * p.k) continue;
      const int ql = e / p.k, j = e - ql * p.k;
      const int64_t m = fg * kRowsPerGroup + ql;
      if (m >= p.M) continue;
      const int64_t o = (m * p.HC + hc) * p.k + j;
      const int id = p.sub_idx[o];
      if (id < 0 || id >= p.n) continue;
      qid[i] = id;
      qrow[i] = ql;
      qval[i] = p.d_sub[o] * Tv * invS;
    }
  }
  auto qstore = [&](int x, int64_t b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kRtQ; ++i)
      if (DQR && qid[i] >= 0 && (qid[i] >> 5) == b) rtile[RT ? x : 0][RT ? qrow[i] : 0][RT ? (qid[i] & 31) : 0] = qval[i];
  };

  const int64_t sb0 = (int64_t)split * p.sblk_per_split;
  const int64_t sb1 = sb0 + p.sblk_per_split < p.sblk ? sb0 + p.sblk_per_split : p.sblk;
  constexpr bool SST = MODE != kModeDiv;
  const bool sst = SST && bal && tid < 32;  // the threads that stage a block's states
  float4 st_next = make_float4(0.f, 0.f, 0.f, 0.f);
  auto sload = [&](int64_t b) __attribute__((always_inline)) {
    if (sst) {
      const int64_t row = b * 32 + tid;
      const int64_t rc = row < nstr ? row : nstr - 1;
      if (MODE == kModeDK)
        st_next = sth[rc];
      else
        st_next.x = cnt[rc];
    }
  };
  auto sstore = [&](int x) __attribute__((always_inline)) {
    if (sst) sstate[SST ? x : 0][SST ? tid : 0] = st_next;
  };
  f32x16 gacc[ND];
#pragma unroll
  for (int db = 0; db < ND; ++db) gacc[db] = f32x16{};
  float usum = 0.f;

  const uint4* sN = p.str + (int64_t)hc * p.sblk * TN;
  const uint4* sT = p.strT + (int64_t)hc * p.sblk * TT;
  Stage<TN> stn;
  Stage<TT> stt;
  if (route) {
    float* rt = &rtile[0][0][0];
    for (int i = tid; i < 2 * kRowsPerGroup * kRtPitch; i += kBalThreads) rt[RT ? i : 0] = 0.f;
    __syncthreads();
    if (sb0 < sb1) {
      rload(sb0);
      rstore(0);
      qstore(0, sb0);
    }
  }
  if (sb0 < sb1) {
    stn.load(sN + sb0 * TN, tid);
    stt.load(sT + sb0 * TT, tid);
    sload(sb0);
    stn.store(tiles[0], tid);
    stt.store(tiles[0] + TN, tid);
    sstore(0);
  }
  __syncthreads();
  for (int64_t sb = sb0; sb < sb1; ++sb) {
    const int cur = (int)((sb - sb0) & 1);
    const bool more = sb + 1 < sb1;
    if (more) {
      stn.load(sN + (sb + 1) * TN, tid);
      stt.load(sT + (sb + 1) * TT, tid);
      sload(sb + 1);
      if (route) rload(sb + 1);
    }
    f32x16 acc = f32x16{};
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      acc = MF::mma(MF::from_vec(tiles[cur][(c / OPV) * kWave + lane], c % OPV), fop[c], acc);
    float gv[16], rtv[16];
    if (route) {
      // this lane's routed entries: key f_loc, queries 8 g4 + 4 par + [0, 4)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        float4* src = (float4*)&rtile[RT ? cur : 0][RT ? f_loc : 0][RT ? 8 * g4 + 4 * par : 0];
        const float4 v = *src;
        *src = make_float4(0.f, 0.f, 0.f, 0.f);
        rtv[4 * g4] = v.x;
        rtv[4 * g4 + 1] = v.y;
        rtv[4 * g4 + 2] = v.z;
        rtv[4 * g4 + 3] = v.w;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = sb * 32 + 8 * (r >> 2) + 4 * par + (r & 3);
      const bool rv = row < nstr;
      const int64_t rc = rv ? row : 0;
      if (DIV) {
        gv[r] = (rv && valid && row != my_f) ? acc[r] : 0.f;
        usum = fmaf(gv[r], gv[r], usum);
        continue;
      }
      float pe, diff;
      if (DK) {
        // d cos / S: balance c p (f - r) T_eff plus the routed d_sub T (q_len)
        float g = route ? rtv[r] : 0.f;
        if (bal) {
          const float4 s = sstate[SST ? cur : 0][SST ? 8 * (r >> 2) + 4 * par + (r & 3) : 0];  // the streamed query's state
          g += exp2f(acc[r] * s.z - s.x) * (ffix - s.y) * (s.z * kLn2) * cc;
        }
        gv[r] = (rv && valid) ? g * invS : 0.f;
        continue;
      } else {
        pe = exp2f(acc[r] * fst.z - fst.x);
        diff = sstate[SST ? cur : 0][SST ? 8 * (r >> 2) + 4 * par + (r & 3) : 0].x * fs - rs_fix;
      }
      if (DQR) {  // c p (f - r) T / S plus the routed d_sub T / S
        gv[r] = (rv && valid) ? __builtin_fmaf(pe * diff, a1, rtv[r]) : 0.f;
        continue;
      }
      gv[r] = (rv && valid) ? pe * diff : 0.f;
      if (!DK) usum = fmaf(gv[r], acc[r], usum);
    }
    typename MF::Op gop[Sh::NOP];
#pragma unroll
    for (int o = 0; o < Sh::NOP; ++o) gop[o] = Ops::from_rows(gv + o * Sh::RPO);
    const uint4* tt = tiles[cur] + TN;
    if (!DIV || grad) {
#pragma unroll
      for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int o = 0; o < Sh::NOP; ++o)
          gacc[db] = MF::mma(MF::from_vec(tt[(db * Sh::TVPD + o / OPV) * kWave + lane], o % OPV), gop[o], gacc[db]);
    }
    if (more) {
      stn.store(tiles[cur ^ 1], tid);
      stt.store(tiles[cur ^ 1] + TN, tid);
      sstore(cur ^ 1);
      if (route) rstore(cur ^ 1);
      qstore(cur ^ 1, sb + 1);
    }
    __syncthreads();
  }

  if (DIV) {
    __shared__ float red[kBalThreads];
    const float wsum = block_sum256(usum, red);
    if (tid == 0) p.u[blockIdx.x] = wsum;
    if (!grad) return;
  }
  // DQ: c T (rho) / sigma * acc; DK: S * acc; Div: coef * acc.  Rows of
  // the output are the fixed rows
  if constexpr (DQR) {
    // d q_hat = S acc; d q = (d q_hat - q_hat (q_hat . d q_hat)) / |q|, as
    // r dy - r^3 (x . dy) x with r = 1 / sqrt(|x|^2 + eps) (lane l holds dims
    // 32 db + 8 g4 + 4 (l/32) + [0, 4) of query l % 32; the partner lane the rest)
    const float S = p.dk_scale[hc];
    const int64_t ro = ((valid ? my_f : 0) * p.HC + hc) * (int64_t)p.half;
    const bool vec = (p.half & 3) == 0;  // whole float4s (the host checks the alignment)
    float xv[ND][16];
    float xdy = 0.f, ss = 0.f;
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * db + 8 * g4 + 4 * par;
        float x[4] = {0.f, 0.f, 0.f, 0.f};
        if (valid && vec && d < p.half) {
          const float4 v = *(const float4*)(p.q_raw + ro + d);
          x[0] = v.x;
          x[1] = v.y;
          x[2] = v.z;
          x[3] = v.w;
        } else if (valid && !vec) {
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = d + i < p.half ? p.q_raw[ro + d + i] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float dy = gacc[db][4 * g4 + i] * S;
          gacc[db][4 * g4 + i] = dy;
          xv[db][4 * g4 + i] = x[i];
          xdy = fmaf(x[i], dy, xdy);
          ss = fmaf(x[i], x[i], ss);
        }
      }
    xdy += partner(xdy, par);
    ss += partner(ss, par);
    const float rr = 1.f / sqrtf(ss + p.eps);
    const float r3x = rr * rr * rr * xdy;
    if (!valid) return;
    float* orow = p.dq + ro;
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * db + 8 * g4 + 4 * par;
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = rr * gacc[db][4 * g4 + i] - r3x * xv[db][4 * g4 + i];
        if (vec) {
          if (d < p.half) *(float4*)(orow + d) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (d + i < p.half) orow[d + i] = o[i];
        }
      }
    return;
  }
  float scale = DIV ? p.coef : (MODE == kModeDK ? p.dk_scale[hc] : cc * Tv / sig);
  if (!DK && p.rho != nullptr) scale *= p.rho[(valid ? my_f : 0) * p.HC + hc];
  if (!DK && p.u != nullptr) {
    const float ut = usum + partner(usum, par);
    if (valid && par == 0) p.u[(int64_t)hc * p.M + my_f] = ut * cc / sig;
  }
  if (!valid) return;
  float* orow = DK ? p.out + (((int64_t)split * p.HC + hc) * p.n + my_f) * p.half
                   : p.out + (my_f * p.HC + hc) * (int64_t)p.half;
  // lane l holds dims 32 db + 8 g4 + 4 (l/32) + [0, 4) in registers 4 g4 + [0, 4)
  const bool vec = (p.half & 3) == 0;  // rows of whole, aligned float4s
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * db + 8 * g4 + 4 * par;
      if (d >= p.half) continue;
      if (vec) {
        *(float4*)(orow + d) = make_float4(gacc[db][4 * g4] * scale, gacc[db][4 * g4 + 1] * scale,
                                           gacc[db][4 * g4 + 2] * scale, gacc[db][4 * g4 + 3] * scale);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (d + i < p.half) orow[d + i] = gacc[db][4 * g4 + i] * scale;
      }
    }
}

// out[i] = sum over s of part[s][i] (part [splits][count]), in split order:
// float4s while count % 4 == 0, else one float per thread.
__global__ __launch_bounds__(256) void split_sum_kernel(const float* __restrict__ part, int splits, int64_t count,
                                                        float* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  if ((count & 3) == 0) {
    const int64_t count4 = count / 4;
    const float4* p4 = (const float4*)part;
    for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < count4; i += stride) {
      float4 s = p4[i];
      for (int k = 1; k < splits; ++k) {
        const float4 v = p4[(int64_t)k * count4 + i];
        s.x += v.x;
        s.y += v.y;
        s.z += v.z;
        s.w += v.w;
      }
      ((float4*)out)[i] = s;
    }
    return;
  }
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < count; i += stride) {
    float s = part[i];
    for (int k = 1; k < splits; ++k) s += part[(int64_t)k * count + i];
    out[i] = s;
  }
}

// dlen[m, hc] = T u (query_scale); part[m, hc] = T rho u (d log_t terms).
// d sub_keys from partial d k_hat slices: dy = sum_i pa[i] + (*gb) sum_i
// pb[i] (each [rows, dim], slices added in order as split_sum_kernel does),
// then the l2 normalisation backward dx = r (dy - y (y . dy)), y = x r,
// r = 1 / sqrt(sum x^2 + eps), in l2norm_bwd_kernel's lanes and order (16
// lanes per row): without pb the result equals split_sum_kernel followed by
// l2norm_bwd_kernel bit for bit.  A workgroup takes 8 rows: the slice sums
// first (one float4 per thread, four slices' loads in flight), staged in
// LDS, then the row pass on 128 of the threads.  dim % 4 == 0, dim <= 128.
__device__ __forceinline__ void add4(float4& a, const float4 b) {
  a.x += b.x;
  a.y += b.y;
  a.z += b.z;
  a.w += b.w;
}

__device__ __forceinline__ float4 slice_sum4(const float4* __restrict__ p, int n, int64_t slice4, int64_t o) {
  float4 a = p[o];
  int i = 1;
  for (; i + 4 <= n; i += 4) {
    const float4 b0 = p[i * slice4 + o], b1 = p[(i + 1) * slice4 + o], b2 = p[(i + 2) * slice4 + o],
                 b3 = p[(i + 3) * slice4 + o];
    add4(a, b0);
    add4(a, b1);
    add4(a, b2);
    add4(a, b3);
  }
  for (; i < n; ++i) add4(a, p[i * slice4 + o]);
  return a;
}

__global__ __launch_bounds__(256) void keys_grad_kernel(const float* __restrict__ x, const float* __restrict__ pa,
                                                        int na, const float* __restrict__ pb, int nb,
                                                        const float* __restrict__ gb, int64_t rows, int dim,
                                                        float eps, float* __restrict__ dx) {
  constexpr int kRows = 8;
  constexpr int kPitch = 144;  // floats per staged row (dim <= 128; rows 16 banks apart)
  __shared__ float tdy[kRows * kPitch];
  const int tid = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * kRows;
  const int d4 = dim >> 2;
  const int64_t slice4 = rows * d4;
  const bool two = pb != nullptr && nb > 0;
  {
    const int rr = tid / d4, c4 = tid - rr * d4;  // d4 <= 32: the block's 8 rows fit 256 threads
    if (rr < kRows && r0 + rr < rows) {
      const int64_t o = (r0 + rr) * d4 + c4;
      float4 a = slice_sum4((const float4*)pa, na, slice4, o);
      if (two) {
        const float g2 = *gb;
        const float4 b = slice_sum4((const float4*)pb, nb, slice4, o);
        a = make_float4(fmaf(g2, b.x, a.x), fmaf(g2, b.y, a.y), fmaf(g2, b.z, a.z), fmaf(g2, b.w, a.w));
      }
      *(float4*)&tdy[rr * kPitch + 4 * c4] = a;
    }
  }
  __syncthreads();
  if (tid >= 16 * kRows) return;
  const int rr = tid >> 4, l = tid & 15;
  const int64_t row = r0 + rr;
  const int64_t rc = row < rows ? row : 0;
  float ss = 0.f, xg = 0.f;
  for (int j = l; j < dim; j += 16) {
    const float v = x[rc * dim + j], g = tdy[rr * kPitch + j];
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
  const float yg = xg * r;
  for (int j = l; j < dim; j += 16) dx[row * dim + j] = r * (tdy[rr * kPitch + j] - x[row * dim + j] * r * yg);
}

__global__ __launch_bounds__(256) void balance_temp_kernel(const float* __restrict__ u, const float* __restrict__ rho,
                                                           int64_t M, int HC, const float* __restrict__ Tp,
                                                           float* __restrict__ dlen, float* __restrict__ part) {
  __shared__ float red[256];
  const float T = *Tp;
  const int64_t total = M * HC;
  float acc = 0.f;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / HC;
    const int hc = (int)(i % HC);
    const float v = u[(int64_t)hc * M + m];
    if (dlen != nullptr) dlen[i] = T * v;
    acc += T * (rho != nullptr ? rho[i] : 1.f) * v;
  }
  const float wsum = block_sum256(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = wsum;
}

__global__ __launch_bounds__(1024) void sum_plain_kernel(const float* __restrict__ x, int64_t n, double scale,
                                                         float* __restrict__ out) {
  __shared__ double part[1024];
  const int tid = threadIdx.x;
  double s = 0.0;
  for (int64_t i = tid; i < n; i += 1024) s += (double)x[i];
  part[tid] = s;
  __syncthreads();
  for (int off = 512; off >= 1; off >>= 1) {
    if (tid < off) part[tid] += part[tid + off];
    __syncthreads();
  }
  if (tid == 0) *out = (float)(part[0] * scale);
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

// fp16 operands are read as 8-dim vectors; fp32 ones one dim per lane.
bool balance_shape_ok(int half, bool f32) {
  return f32 ? (half >= 1 && half <= 128) : (half >= 8 && half <= 128 && half % 8 == 0);
}

// Host view of BalShape: the padded width and the 16-byte vectors per lane
// of a 32-row block in the normal and transposed packs.
struct PackDims {
  int HP, NV, ND, TVPD;
};

PackDims pack_dims(int half, bool f32) {
  PackDims d;
  d.HP = f32 ? KeyPack<float>::padded_half(half) : KeyPack<_Float16>::padded_half(half);
  d.NV = f32 ? KeyPack<float>::vectors_per_lane(d.HP) : KeyPack<_Float16>::vectors_per_lane(d.HP);
  d.ND = (d.HP + 31) / 32;
  d.TVPD = f32 ? 4 : 2;
  return d;
}

// MACRO(E, HP) for the precision and padded width of a launch.
#define MPL_BAL_DISPATCH(F32, HPV, MACRO) \
  do {                                     \
    if (F32) {                             \
      switch (HPV) {                       \
        case 8: MACRO(float, 8); break;    \
        case 16: MACRO(float, 16); break;  \
        case 32: MACRO(float, 32); break;  \
        case 64: MACRO(float, 64); break;  \
        default: MACRO(float, 128); break; \
      }                                    \
    } else {                               \
      switch (HPV) {                       \
        case 16: MACRO(_Float16, 16); break;  \
        case 32: MACRO(_Float16, 32); break;  \
        case 64: MACRO(_Float16, 64); break;  \
        default: MACRO(_Float16, 128); break; \
      }                                    \
    }                                      \
  } while (0)

unsigned grid_for(int64_t items, int64_t per_block, unsigned cap = 4096) {
  int64_t g = cdiv(items, per_block);
  if (g < 1) g = 1;
  return (unsigned)(g < cap ? g : cap);
}

struct DivLayout {
  size_t kt, part, lpart, total;
  PackDims pd;
  int splits;
  int64_t nblk, sbps, groups;
};

DivLayout div_layout(int H, int n, int half, bool f32) {
  DivLayout L;
  const int HC = 2 * H;
  L.pd = pack_dims(half, f32);
  L.nblk = cdiv(n, 32);
  const int64_t kgroups = (int64_t)HC * cdiv(n, kRowsPerGroup);
  int64_t sp = cdiv(512, kgroups);
  if (sp > L.nblk) sp = L.nblk;
  if (sp < 1) sp = 1;
  L.sbps = cdiv(L.nblk, sp);
  L.splits = (int)cdiv(L.nblk, L.sbps);
  L.groups = kgroups * L.splits;
  size_t o = 0;
  L.kt = o;
  o += al256((size_t)HC * L.nblk * L.pd.ND * L.pd.TVPD * kWave * 16);
  L.part = o;
  o += al256((size_t)L.splits * HC * n * half * 4);
  L.lpart = o;
  o += al256((size_t)L.groups * 4);
  L.total = o;
  return L;
}


struct BwdLayout {
  size_t qn, qt, kt, sigma, dks, mx, part, u, tpart, total;
  PackDims pd;
  int splits, mx_groups;
  int64_t mblk, nblk, sbps, mx_tpg;
};

BwdLayout bwd_layout(int64_t M, int H, int n, int half, bool f32) {
  BwdLayout L;
  const int HC = 2 * H;
  L.pd = pack_dims(half, f32);
  L.mblk = cdiv(M, 32);
  L.nblk = cdiv(n, 32);
  // the sub-key-side pass: HC * ceil(n / 128) workgroups, the query range
  // split so that about 512 run
  const int64_t kgroups = (int64_t)HC * cdiv(n, kRowsPerGroup);
  int64_t sp = cdiv(512, kgroups);
  if (sp > L.mblk) sp = L.mblk;
  if (sp < 1) sp = 1;
  L.sbps = cdiv(L.mblk, sp);
  L.splits = (int)cdiv(L.mblk, L.sbps);
  const size_t tvec = (size_t)L.pd.ND * L.pd.TVPD * kWave * 16;  // bytes per block of a transposed pack
  size_t o = 0;
  L.qn = o;
  o += al256((size_t)HC * L.mblk * L.pd.NV * kWave * 16);
  L.qt = o;
  o += al256((size_t)HC * L.mblk * tvec);
  L.kt = o;
  o += al256((size_t)HC * L.nblk * tvec);
  L.sigma = o;
  o += al256((size_t)HC * 4);
  L.dks = o;
  o += al256((size_t)HC * 4);
  L.mx_tpg = cdiv(M > 0 ? M : 1, 256) < 64 ? 64 : cdiv(M, 256);  // about 256 workgroups of partial maxima
  L.mx_groups = (int)cdiv(M > 0 ? M : 1, L.mx_tpg);
  L.mx = o;
  o += al256((size_t)L.mx_groups * HC * 8);
  L.part = o;
  o += al256((size_t)L.splits * HC * n * half * 4);
  L.u = o;
  o += al256((size_t)HC * M * 4);
  L.tpart = o;
  o += al256((size_t)HC * M * 4);
  L.total = o;
  return L;
}

template <bool TRANS>
void launch_pack(const PackDims& pd, bool f32, const float* X, int64_t s_hc, int64_t s_row, int64_t nrows, int HC,
                 int half, const float* scale, int64_t sc_hc, int64_t sc_row, int64_t nblk, uint4* out,
                 hipStream_t s) {
  const int64_t total = (int64_t)HC * nblk * (TRANS ? pd.ND * pd.TVPD : pd.NV) * kWave;
  const unsigned g = grid_for(total, 256, 8192);
#define MPL_PACK(EV, HPV) \
  pack_rows_kernel<TRANS, EV, HPV><<<g, 256, 0, s>>>(X, s_hc, s_row, nrows, HC, half, scale, sc_hc, sc_row, nblk, out)
  MPL_BAL_DISPATCH(f32, pd.HP, MPL_PACK);
#undef MPL_PACK
}

}  // namespace
}  // namespace mpl

using namespace mpl;

extern "C" int mpl_route_counts(const int32_t* slots, const int32_t* clean_sub_idx, int64_t M, int H, int n, int k,
                                float* subkey_counts, float* clean_counts, float* slot_counts, void* stream) {
  clear_error();
  MPL_REQUIRE(M >= 0 && H >= 1 && n >= 1 && k >= 1 && k <= n, MPL_EINVAL, "mpl_route_counts: bad shape");
  MPL_REQUIRE(M == 0 || slots != nullptr || (subkey_counts == nullptr && slot_counts == nullptr), MPL_EINVAL,
              "mpl_route_counts: slots is null");
  MPL_REQUIRE(clean_counts == nullptr || M == 0 || clean_sub_idx != nullptr, MPL_EINVAL,
              "mpl_route_counts: clean_counts needs clean_sub_idx");
  hipStream_t s = (hipStream_t)stream;
  const int64_t hn = (int64_t)H * 2 * n;
  {
    const int64_t na = subkey_counts ? hn : 0, nb = clean_counts ? hn : 0;
    const int64_t nc = slot_counts ? (int64_t)n * n : 0;
    if (na + nb + nc > 0)
      fill_zero3_kernel<<<grid_for(na + nb + nc, 256), 256, 0, s>>>(subkey_counts, na, clean_counts, nb,
                                                                     slot_counts, nc);
  }
  if (M > 0 && (subkey_counts || clean_counts || slot_counts)) {
    const int use_lds = n <= 4096 ? 1 : 0;
    // tokens per workgroup with LDS histograms: the 4n-bin flush against
    // the 3k ids per token, at 2n/k tokens (n = 512, k = 16: 64 tokens,
    // 37.8 us against 41.6 us at 16n/3k for 8,192 tokens)
    int64_t tpg = use_lds ? cdiv(2 * (int64_t)n, (int64_t)k) : 32;
    if (tpg < 64) tpg = 64;
    const int64_t min_tpg = cdiv(M * H, 2048);
    if (tpg < min_tpg) tpg = min_tpg;
    const int64_t groups = (int64_t)H * cdiv(M, tpg);
    MPL_REQUIRE(tpg * 2 * k < ((int64_t)1 << 31), MPL_EUNSUPPORTED, "mpl_route_counts: k too large");
    const bool p2 = (k & (k - 1)) == 0 && (n & (n - 1)) == 0;
    const int kshift = p2 ? __builtin_ctz((unsigned)k) : 0, nshift = p2 ? __builtin_ctz((unsigned)n) : 0;
#define MPL_RC(P) \
  route_counts_kernel<P><<<(unsigned)groups, 256, use_lds ? 16 * n : 0, s>>>( \
      slots, clean_sub_idx, M, H, n, k, kshift, nshift, tpg, use_lds, subkey_counts, clean_counts, slot_counts)
    if (p2) MPL_RC(true);
    else MPL_RC(false);
#undef MPL_RC
  }
  return check_launch("mpl_route_counts");
}

static int64_t fwd_groups(int64_t M, int H) { return (int64_t)2 * H * cdiv(M, kRowsPerGroup); }

extern "C" size_t mpl_balance_state_bytes(int64_t M, int H) {
  if (M <= 0 || H <= 0) return 0;
  return (size_t)M * 2 * H * 16 + (size_t)fwd_groups(M, H) * 4;
}

extern "C" int mpl_balance_fwd(const float* queries, int scaled, const void* packed_keys, const float* clean_counts,
                               int64_t M, int H, int n, int half, int k, int score_dtype, const float* temperature,
                               void* state, float* loss, void* stream) {
  clear_error();
  MPL_REQUIRE(M >= 0 && H >= 1 && n >= 1 && k >= 1 && k <= n, MPL_EINVAL, "mpl_balance_fwd: bad shape");
  MPL_REQUIRE(score_dtype == MPL_F16 || score_dtype == MPL_F32, MPL_EINVAL, "mpl_balance_fwd: bad score_dtype %d",
              score_dtype);
  const bool f32 = score_dtype == MPL_F32;
  MPL_REQUIRE(balance_shape_ok(half, f32), MPL_EUNSUPPORTED,
              "mpl_balance_fwd: %s scoring needs %s (half = %d)", f32 ? "fp32" : "fp16",
              f32 ? "half <= 128" : "half %% 8 == 0 and half <= 128", half);
  MPL_REQUIRE(loss != nullptr && (M == 0 || (queries && packed_keys && clean_counts && state && temperature)),
              MPL_EINVAL, "mpl_balance_fwd: null buffer");
  hipStream_t s = (hipStream_t)stream;
  const int HC = 2 * H;
  if (M == 0) {  // f = counts / (M k) and the mean over tokens are 0/0 (memory.py:208-213)
    fill_value_kernel<<<1, 64, 0, s>>>(loss, 1, __builtin_nanf(""));
    return check_launch("mpl_balance_fwd");
  }
  BalFwdParams p;
  p.q = queries;
  p.packed = (const uint4*)packed_keys;
  p.counts = clean_counts;
  p.inv_mk = (float)(1.0 / ((double)M * k));
  p.T = temperature;
  p.scaled = scaled ? 1 : 0;
  p.M = M;
  p.HC = HC;
  p.n = n;
  p.half = half;
  p.nblk = (int)cdiv(n, 32);
  p.state = (float4*)state;
  p.parts = (float*)((float4*)state + M * HC);
  const unsigned grid = (unsigned)fwd_groups(M, H);
#define MPL_FWD(EV, HPV) balance_fwd_kernel<EV, HPV><<<grid, kBalThreads, 0, s>>>(p)
  MPL_BAL_DISPATCH(f32, pack_dims(half, f32).HP, MPL_FWD);
#undef MPL_FWD
  balance_loss_kernel<<<1, 1024, 0, s>>>(p.parts, grid, (float)((double)n / ((double)HC * M)), loss);
  return check_launch("mpl_balance_fwd");
}

extern "C" size_t mpl_lookup_bwd_dense_workspace_bytes(int64_t M, int H, int n, int half, int score_dtype) {
  const bool f32 = score_dtype == MPL_F32;
  if (M < 0 || H < 1 || n < 1 || (score_dtype != MPL_F16 && !f32) || !balance_shape_ok(half, f32)) return 0;
  return bwd_layout(M, H, n, half, f32).total;
}

// The fused form's sub-key gradient: d sub_keys [2H, n, half] written from
// the sub-key pass's slices (and, with g_div, the key diversity pass's,
// whose loss goes to div_loss), through the l2 normalisation of sub_keys.
struct KeysGradArgs {
  const float* sub_keys;
  const float* g_div;
  void* div_ws;
  float* div_loss;
  float* d_sub_keys;
};

// q_raw / d_queries (both or neither): the fused form (kModeDQR) that also
// takes the routed d q_hat and the normalisation backward, writing d queries
// instead of the balance d q_hat.
static int lookup_bwd_dense_impl(const float* q_hat, const float* q_len, const float* k_hat,
                                 const void* packed_keys, const int32_t* sub_idx, const float* d_sub,
                                 const float* clean_counts, const void* state, const float* g_balance,
                                 int balance_temperature_grad, int query_scale, int64_t M, int H, int n, int half,
                                 int k, int score_dtype, const float* temperature, void* workspace,
                                 size_t workspace_bytes, float* dq_hat, float* dk_hat, float* dlen, float* dlogt,
                                 const float* q_raw, float eps, float* d_queries, const KeysGradArgs* kg,
                                 int phase, void* stream) {
  MPL_REQUIRE(M >= 0 && H >= 1 && n >= 1 && k >= 1 && k <= n, MPL_EINVAL, "mpl_lookup_bwd_dense: bad shape");
  MPL_REQUIRE(score_dtype == MPL_F16 || score_dtype == MPL_F32, MPL_EINVAL,
              "mpl_lookup_bwd_dense: bad score_dtype %d", score_dtype);
  const bool f32 = score_dtype == MPL_F32;
  MPL_REQUIRE(balance_shape_ok(half, f32), MPL_EUNSUPPORTED,
              "mpl_lookup_bwd_dense: %s scoring needs %s (half = %d)", f32 ? "fp32" : "fp16",
              f32 ? "half <= 128" : "half %% 8 == 0 and half <= 128", half);
  const bool bal = g_balance != nullptr;
  const bool routed = sub_idx != nullptr || d_sub != nullptr;
  const bool btg = bal && balance_temperature_grad != 0;
  const bool scaled = btg && query_scale != 0;
  const bool fused = d_queries != nullptr;
  if (fused) {
    MPL_REQUIRE(M > 0 && bal && sub_idx != nullptr && d_sub != nullptr && q_raw != nullptr, MPL_EINVAL,
                "mpl_lookup_bwd_dense_queries: needs tokens, the balance term, the routed term and the queries");
    MPL_REQUIRE(!btg && query_scale == 0 && k <= 16, MPL_EUNSUPPORTED,
                "mpl_lookup_bwd_dense_queries: only without query_scale and balance_temperature_grad, k <= 16");
    MPL_REQUIRE((half & 3) != 0 || ((uintptr_t)q_raw & 15) == 0, MPL_EINVAL,
                "mpl_lookup_bwd_dense_queries: queries must be 16-byte aligned");
  }
  MPL_REQUIRE((dk_hat != nullptr || kg != nullptr) && (!btg || dlogt != nullptr), MPL_EINVAL,
              "mpl_lookup_bwd_dense: null output");
  MPL_REQUIRE(!routed || (sub_idx != nullptr && d_sub != nullptr), MPL_EINVAL,
              "mpl_lookup_bwd_dense: sub_idx and d_sub go together");
  MPL_REQUIRE(M == 0 || q_len != nullptr || !(query_scale != 0 && (routed || scaled)), MPL_EINVAL,
              "mpl_lookup_bwd_dense: q_len needed with query_scale");
  hipStream_t s = (hipStream_t)stream;
  const int HC = 2 * H;
  if (M == 0 || (!bal && !routed)) {
    fill_zero_kernel<<<grid_for((int64_t)HC * n * half, 256), 256, 0, s>>>(dk_hat, (int64_t)HC * n * half);
    if (btg) fill_zero_kernel<<<1, 256, 0, s>>>(dlogt, 1);
    if (bal && dq_hat != nullptr && M > 0)
      fill_zero_kernel<<<grid_for(M * HC * half, 256), 256, 0, s>>>(dq_hat, M * HC * half);
    return check_launch("mpl_lookup_bwd_dense");
  }
  MPL_REQUIRE((q_hat || fused) && k_hat && packed_keys && temperature, MPL_EINVAL,
              "mpl_lookup_bwd_dense: null buffer");
  MPL_REQUIRE(!bal || (clean_counts && state && (dq_hat || fused)), MPL_EINVAL,
              "mpl_lookup_bwd_dense: the balance term needs clean_counts, state and dq_hat");
  const BwdLayout L = bwd_layout(M, H, n, half, f32);
  MPL_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, MPL_EWORKSPACE,
              "mpl_lookup_bwd_dense: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
  char* ws = (char*)workspace;
  uint4* qn = (uint4*)(ws + L.qn);
  uint4* qt = (uint4*)(ws + L.qt);
  uint4* kt = (uint4*)(ws + L.kt);
  float* sigma = (float*)(ws + L.sigma);
  float* dks = (float*)(ws + L.dks);
  float2* mx = (float2*)(ws + L.mx);
  float* part = (float*)(ws + L.part);
  float* u = (float*)(ws + L.u);
  float* tpart = (float*)(ws + L.tpart);
  const float* rho = scaled ? q_len : nullptr;

  // phase 1: the packs, scales and query pass; phase 2: the sub-key passes,
  // from what phase 1 left in the same workspace; 0: both
  const bool run_q = phase != 2, run_k = phase != 1;
  // without q_hat (fused form only) the packs normalise the raw queries
  const bool norm = q_hat == nullptr;
  const float* qsrc = norm ? q_raw : q_hat;
  const bool both = !f32 && L.pd.HP == half && (half == 64 || half == 128) && ((uintptr_t)qsrc & 15) == 0;
  MPL_REQUIRE(both || !norm, MPL_EINVAL, "mpl_lookup_bwd_dense: q_hat is needed here (only fp16 scoring at half "
              "64 or 128 packs the raw queries)");
#define MPL_PACK_BOTH(HPV, NRM)                                                                               \
  pack_rows_both_f16_kernel<HPV, NRM><<<(unsigned)(HC * L.mblk), 256, 0, s>>>(qsrc, half, (int64_t)HC * half, M, \
                                                                              L.mblk, eps, qn, qt)
  if (!run_q) {
  } else if (both && half == 128) {
    if (norm) MPL_PACK_BOTH(128, true);
    else MPL_PACK_BOTH(128, false);
  } else if (both) {
    if (norm) MPL_PACK_BOTH(64, true);
    else MPL_PACK_BOTH(64, false);
  }
#undef MPL_PACK_BOTH
  if (run_q && !both) {
    launch_pack<false>(L.pd, f32, q_hat, half, (int64_t)HC * half, M, HC, half, nullptr, 0, 0, L.mblk, qn, s);
    launch_pack<true>(L.pd, f32, q_hat, half, (int64_t)HC * half, M, HC, half, nullptr, 0, 0, L.mblk, qt, s);
  }
  if (run_q && bal)
    launch_pack<true>(L.pd, f32, k_hat, (int64_t)n * half, half, n, HC, half, nullptr, 0, 0, L.nblk, kt, s);
  const float inv_mk = (float)(1.0 / ((double)M * k));
  const float coef = (float)((double)n / ((double)HC * M));
  const int vpt = HC * k / 4;
  if (!run_q) {
  } else if (k % 4 == 0 && 256 % vpt == 0 && 256 % HC == 0 && ((uintptr_t)d_sub & 15) == 0)
    bwd_max_vec_kernel<<<L.mx_groups, 256, 0, s>>>(routed ? d_sub : nullptr, query_scale ? q_len : nullptr, M, HC,
                                                   k, L.mx_tpg, mx);
  else
    bwd_max_kernel<<<L.mx_groups, 256, 0, s>>>(routed ? d_sub : nullptr, query_scale ? q_len : nullptr, M, HC, k,
                                               L.mx_tpg, mx);
  if (run_q)
    bwd_scale_kernel<<<HC, 256, 0, s>>>(bal ? clean_counts : nullptr, mx, L.mx_groups, n, HC, inv_mk,
                                      bal ? g_balance : nullptr, coef, temperature, btg ? 1 : 0, query_scale ? 1 : 0,
                                      bal ? sigma : nullptr, dks);

  BalGradParams p = {};
  p.state = (const float4*)state;
  p.counts = clean_counts;
  p.sigma = sigma;
  p.g = g_balance;
  p.inv_mk = inv_mk;
  p.coef = coef;
  p.T = temperature;
  p.M = M;
  p.HC = HC;
  p.n = n;
  p.half = half;
  p.rho = rho;

  // d q_hat (balance term): fixed = queries, streamed = sub-keys
  BalGradParams pq = p;
  pq.fix = qn;
  pq.str = (const uint4*)packed_keys;
  pq.strT = kt;
  pq.fblk = L.mblk;
  pq.sblk = L.nblk;
  pq.splits = 1;
  pq.sblk_per_split = L.nblk;
  pq.out = dq_hat;
  pq.u = btg ? u : nullptr;
  if (fused) {
    pq.out = nullptr;
    pq.u = nullptr;
    pq.sub_idx = sub_idx;
    pq.d_sub = d_sub;
    pq.k = k;
    pq.dk_scale = dks;
    pq.q_raw = q_raw;
    pq.eps = eps;
    pq.dq = d_queries;
  }
  const unsigned gq = (unsigned)(HC * cdiv(M, kRowsPerGroup));
  // d k_hat (balance and routed terms): fixed = sub-keys, streamed = queries
  BalGradParams pk = p;
  pk.fix = (const uint4*)packed_keys;
  pk.str = qn;
  pk.strT = qt;
  pk.fblk = L.nblk;
  pk.sblk = L.mblk;
  pk.splits = L.splits;
  pk.sblk_per_split = L.sbps;
  pk.out = (L.splits == 1 && kg == nullptr) ? dk_hat : part;
  pk.u = nullptr;
  pk.rho = nullptr;
  pk.bal = bal ? 1 : 0;
  pk.sub_idx = routed ? sub_idx : nullptr;
  pk.d_sub = d_sub;
  pk.qlen_rt = query_scale ? q_len : nullptr;
  pk.k = k;
  pk.dk_scale = dks;
  const unsigned gk = (unsigned)(HC * cdiv(n, kRowsPerGroup) * L.splits);
#define MPL_GRAD(EV, HPV)                                                                            \
  if (run_q && fused) balance_grad_kernel<kModeDQR, EV, HPV><<<gq, kBalThreads, 0, s>>>(pq);         \
  else if (run_q && bal) balance_grad_kernel<kModeDQ, EV, HPV><<<gq, kBalThreads, 0, s>>>(pq);       \
  if (run_k) balance_grad_kernel<kModeDK, EV, HPV><<<gk, kBalThreads, 0, s>>>(pk)
  MPL_BAL_DISPATCH(f32, L.pd.HP, MPL_GRAD);
#undef MPL_GRAD
  if (!run_k) return check_launch("mpl_lookup_bwd_dense");
  if (kg != nullptr) {
    // d sub_keys straight from the slices: the sub-key pass's, and with
    // g_div the key diversity Gram pass's on the same packs (memory.py:230-240)
    float* dpart = nullptr;
    int dsplits = 0;
    if (kg->g_div != nullptr) {
      const DivLayout Ld = div_layout(H, n, half, f32);
      dpart = (float*)((char*)kg->div_ws + Ld.part);
      float* lpart = (float*)((char*)kg->div_ws + Ld.lpart);
      const double D = (double)HC * n * (double)(n - 1);
      BalGradParams pd = {};
      pd.fix = (const uint4*)packed_keys;
      pd.str = (const uint4*)packed_keys;
      pd.strT = kt;
      pd.coef = (float)(4.0 / D);
      pd.M = 0;
      pd.HC = HC;
      pd.n = n;
      pd.half = half;
      pd.fblk = L.nblk;
      pd.sblk = L.nblk;
      pd.splits = Ld.splits;
      pd.sblk_per_split = Ld.sbps;
      pd.out = dpart;
      pd.u = lpart;
      const unsigned gd = (unsigned)Ld.groups;
#define MPL_DIV(EV, HPV) balance_grad_kernel<kModeDiv, EV, HPV><<<gd, kBalThreads, 0, s>>>(pd)
      MPL_BAL_DISPATCH(f32, L.pd.HP, MPL_DIV);
#undef MPL_DIV
      sum_plain_kernel<<<1, 1024, 0, s>>>(lpart, Ld.groups, 1.0 / D, kg->div_loss);
      dsplits = Ld.splits;
    }
    const int64_t rows = (int64_t)HC * n;
    keys_grad_kernel<<<(unsigned)cdiv(rows, 8), 256, 0, s>>>(kg->sub_keys, part, L.splits, dpart, dsplits, kg->g_div,
                                                             rows, half, eps, kg->d_sub_keys);
  } else if (L.splits > 1) {
    const int64_t cnt = (int64_t)HC * n * half;
    split_sum_kernel<<<grid_for(cnt, 256), 256, 0, s>>>(part, L.splits, cnt, dk_hat);
  }
  if (btg) {
    const unsigned gt = grid_for(M * HC, 256);
    balance_temp_kernel<<<gt, 256, 0, s>>>(u, rho, M, HC, temperature, query_scale ? dlen : nullptr, tpart);
    sum_plain_kernel<<<1, 1024, 0, s>>>(tpart, gt, 1.0, dlogt);
  }
  return check_launch("mpl_lookup_bwd_dense");
}

extern "C" int mpl_lookup_bwd_dense(const float* q_hat, const float* q_len, const float* k_hat,
                                    const void* packed_keys, const int32_t* sub_idx, const float* d_sub,
                                    const float* clean_counts, const void* state, const float* g_balance,
                                    int balance_temperature_grad, int query_scale, int64_t M, int H, int n,
                                    int half, int k, int score_dtype, const float* temperature, void* workspace,
                                    size_t workspace_bytes, float* dq_hat, float* dk_hat, float* dlen, float* dlogt,
                                    void* stream) {
  clear_error();
  return lookup_bwd_dense_impl(q_hat, q_len, k_hat, packed_keys, sub_idx, d_sub, clean_counts, state, g_balance,
                               balance_temperature_grad, query_scale, M, H, n, half, k, score_dtype, temperature,
                               workspace, workspace_bytes, dq_hat, dk_hat, dlen, dlogt, nullptr, 0.f, nullptr,
                               nullptr, 0, stream);
}

extern "C" int mpl_lookup_bwd_dense_queries(const float* q_hat, const float* queries, const float* k_hat,
                                            const void* packed_keys, const int32_t* sub_idx, const float* d_sub,
                                            const float* clean_counts, const void* state, const float* g_balance,
                                            int64_t M, int H, int n, int half, int k, int score_dtype,
                                            const float* temperature, void* workspace, size_t workspace_bytes,
                                            float eps, float* d_queries, const float* sub_keys,
                                            const float* g_diversity, void* div_workspace,
                                            size_t div_workspace_bytes, float* diversity_loss, float* d_sub_keys,
                                            int phase, void* stream) {
  clear_error();
  MPL_REQUIRE(phase >= 0 && phase <= 2, MPL_EINVAL, "mpl_lookup_bwd_dense_queries: phase must be 0, 1 or 2");
  MPL_REQUIRE(d_queries != nullptr && sub_keys != nullptr && d_sub_keys != nullptr, MPL_EINVAL,
              "mpl_lookup_bwd_dense_queries: null d_queries, sub_keys or d_sub_keys");
  MPL_REQUIRE(half <= 128 && half % 4 == 0, MPL_EUNSUPPORTED,
              "mpl_lookup_bwd_dense_queries: half must be a multiple of 4 up to 128");
  if (g_diversity != nullptr) {
    const size_t need = mpl_key_diversity_workspace_bytes(H, n, half, score_dtype);
    MPL_REQUIRE(need > 0 && n > 1 && diversity_loss != nullptr && div_workspace != nullptr &&
                    div_workspace_bytes >= need,
                MPL_EWORKSPACE, "mpl_lookup_bwd_dense_queries: key diversity needs n > 1, its loss output and a "
                "workspace of %zu bytes (%zu given)", need, div_workspace_bytes);
  }
  const KeysGradArgs kg{sub_keys, g_diversity, div_workspace, diversity_loss, d_sub_keys};
  return lookup_bwd_dense_impl(q_hat, nullptr, k_hat, packed_keys, sub_idx, d_sub, clean_counts, state, g_balance,
                               0, 0, M, H, n, half, k, score_dtype, temperature, workspace, workspace_bytes,
                               nullptr, nullptr, nullptr, nullptr, queries, eps, d_queries, &kg, phase, stream);
}

namespace mpl {
namespace {

}  // namespace
}  // namespace mpl

extern "C" size_t mpl_key_diversity_workspace_bytes(int H, int n, int half, int score_dtype) {
  const bool f32 = score_dtype == MPL_F32;
  if (H < 1 || n < 1 || (score_dtype != MPL_F16 && !f32) || !balance_shape_ok(half, f32)) return 0;
  return div_layout(H, n, half, f32).total;
}

extern "C" int mpl_key_diversity(const float* k_hat, const void* packed_keys, int H, int n, int half,
                                 int score_dtype, void* workspace, size_t workspace_bytes, float* loss,
                                 float* d_k_hat, void* stream) {
  clear_error();
  MPL_REQUIRE(H >= 1 && n >= 1, MPL_EINVAL, "mpl_key_diversity: bad shape");
  MPL_REQUIRE(score_dtype == MPL_F16 || score_dtype == MPL_F32, MPL_EINVAL, "mpl_key_diversity: bad score_dtype %d",
              score_dtype);
  const bool f32 = score_dtype == MPL_F32;
  MPL_REQUIRE(balance_shape_ok(half, f32), MPL_EUNSUPPORTED, "mpl_key_diversity: %s Gram tiles need %s (half = %d)",
              f32 ? "fp32" : "fp16", f32 ? "half <= 128" : "half %% 8 == 0 and half <= 128", half);
  MPL_REQUIRE(k_hat && packed_keys && loss, MPL_EINVAL, "mpl_key_diversity: null buffer");
  const DivLayout L = div_layout(H, n, half, f32);
  MPL_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, MPL_EWORKSPACE,
              "mpl_key_diversity: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  const int HC = 2 * H;
  char* ws = (char*)workspace;
  uint4* kt = (uint4*)(ws + L.kt);
  float* part = (float*)(ws + L.part);
  float* lpart = (float*)(ws + L.lpart);
  launch_pack<true>(L.pd, f32, k_hat, (int64_t)n * half, half, n, HC, half, nullptr, 0, 0, L.nblk, kt, s);
  // D = H * 2 * n * (n - 1) (memory.py:240); n = 1 gives 0/0 as the reference
  const double D = (double)HC * n * (double)(n - 1);
  BalGradParams p = {};
  p.fix = (const uint4*)packed_keys;
  p.str = (const uint4*)packed_keys;
  p.strT = kt;
  p.coef = (float)(4.0 / D);
  p.M = 0;
  p.HC = HC;
  p.n = n;
  p.half = half;
  p.fblk = L.nblk;
  p.sblk = L.nblk;
  p.splits = L.splits;
  p.sblk_per_split = L.sbps;
  p.out = d_k_hat == nullptr ? nullptr : (L.splits == 1 ? d_k_hat : part);
  p.u = lpart;
  const unsigned g = (unsigned)L.groups;
#define MPL_DIV(EV, HPV) balance_grad_kernel<kModeDiv, EV, HPV><<<g, kBalThreads, 0, s>>>(p)
  MPL_BAL_DISPATCH(f32, L.pd.HP, MPL_DIV);
#undef MPL_DIV
  if (d_k_hat != nullptr && L.splits > 1) {
    const int64_t cnt = (int64_t)HC * n * half;
    split_sum_kernel<<<grid_for(cnt, 256), 256, 0, s>>>(part, L.splits, cnt, d_k_hat);
  }
  sum_plain_kernel<<<1, 1024, 0, s>>>(lpart, L.groups, 1.0 / D, loss);
  return check_launch("mpl_key_diversity");
}

namespace mpl {
namespace {

// revive_dead_keys (memory.py:243-281), one workgroup per codebook, in place:
// keys whose usage is below threshold / n become the normalised picked query
// plus noise * normal, their usage 1/n, and the codebook's usage is divided
// by its new sum (fp64, fixed order).
__global__ __launch_bounds__(256) void revive_kernel(float* __restrict__ keys, float* __restrict__ usage,
                                                     const float* __restrict__ queries, int64_t M,
                                                     const int32_t* __restrict__ pick,
                                                     const float* __restrict__ normal, int HC, int n, int half,
                                                     float threshold, float noise, uint8_t* __restrict__ dead) {
  __shared__ double part[256];
  const int tid = threadIdx.x;
  const int hc = blockIdx.x;
  float* u = usage + (int64_t)hc * n;
  const float lim = threshold / (float)n;
  const float inv_n = 1.0f / (float)n;
  double s = 0.0;
  for (int i = tid; i < n; i += 256) {
    const float v = u[i];
    s += (double)(v < lim ? inv_n : v);
  }
  part[tid] = s;
  __syncthreads();
  for (int off = 128; off >= 1; off >>= 1) {
    if (tid < off) part[tid] += part[tid + off];
    __syncthreads();
  }
  const float total = (float)part[0];
  // keys: 16 lanes per row
  const int l = tid & 15;
  for (int i0 = 0; i0 < n; i0 += 16) {
    const int i = i0 + (tid >> 4);
    const bool is_dead = i < n && u[i < n ? i : 0] < lim;  // wave-divergent, no barrier inside
    if (!is_dead) continue;
    int pk = pick[(int64_t)hc * n + i];
    pk = pk < 0 ? 0 : (pk >= M ? (int)(M - 1) : pk);
    const float* qr = queries + ((int64_t)pk * HC + hc) * half;
    const float* zr = normal + ((int64_t)hc * n + i) * half;
    float* kr = keys + ((int64_t)hc * n + i) * half;
    float ss = 0.f;
    for (int d = l; d < half; d += 16) {
      const float x = fmaf(noise, zr[d], qr[d]);
      ss = fmaf(x, x, ss);
    }
    // the 16 lanes of this row are contiguous and all take this branch
    for (int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 16);
    const float r = 1.0f / sqrtf(ss + 1e-6f);
    for (int d = l; d < half; d += 16) kr[d] = fmaf(noise, zr[d], qr[d]) * r;
  }
  __syncthreads();  // every row read the old usage
  for (int i = tid; i < n; i += 256) {
    const float v = u[i];
    const bool dd = v < lim;
    u[i] = (dd ? inv_n : v) / total;
    if (dead != nullptr) dead[(int64_t)hc * n + i] = dd ? 1 : 0;
  }
}

}  // namespace
}  // namespace mpl

extern "C" int mpl_revive_keys(float* sub_keys, float* subkey_usage, const float* queries, int64_t M,
                               const int32_t* pick, const float* normal, int H, int n, int half, float threshold,
                               float noise, uint8_t* dead, void* stream) {
  clear_error();
  MPL_REQUIRE(H >= 1 && n >= 1 && half >= 1 && M >= 1, MPL_EINVAL, "mpl_revive_keys: bad shape");
  MPL_REQUIRE(sub_keys && subkey_usage && queries && pick && normal, MPL_EINVAL, "mpl_revive_keys: null buffer");
  revive_kernel<<<2 * H, 256, 0, (hipStream_t)stream>>>(sub_keys, subkey_usage, queries, M, pick, normal, 2 * H, n,
                                                        half, threshold, noise, dead);
  return check_launch("mpl_revive_keys");
}
