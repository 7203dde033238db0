// Backward of the memory-layer lookup (XLA's derivative of memory.py:136-193,
// written out; the routing selection is piecewise constant, so gradients flow
// through the selected clean scores, the softmax and the gather).
//
//   route:   dw[m,r]   = <g_out[m], values[read[m,r]]>           (memory.py:192)
//            ds[m,h,j] = w (dw - sum_j w dw)                      (softmax, :178)
//            d_sub[m,h,c,i] = sum_j ds[m,h,j] [rank_c(j) == i]    (:167-175)
//            d_log_t  += d_sub * sub_scores  (T = exp(log_t) with the
//                        straight-through clamp of :143-146, so dT/dlog_t = T)
//   queries: dq_hat = sum_i d_sub_i * T * q_len * k_hat[sub_idx_i] (+ dense
//            part), then the l2-normalisation backward (:30-31, :136-137)
//   keys:    dk_hat[key] = sum over (m,i) with sub_idx == key of
//            d_sub * T * q_len * q_hat[m]: a deterministic sort-by-key
//            segmented sum (the row merge of rows.hip), then the
//            l2-normalisation backward.
#include <math.h>

#include "common.h"


namespace mpl {

constexpr int kBwdThreads = 256;
constexpr int kMaxRows = 128;  // H * k per token

template <typename V>
struct RowLoad;
template <>
struct RowLoad<_Float16> {
  static constexpr int kElems = 8;
  __device__ static void unpack(uint4 u, float* f) {
    const half8 h = __builtin_bit_cast(half8, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)h[i];
  }
};
template <>
struct RowLoad<float> {
  static constexpr int kElems = 4;
  __device__ static void unpack(uint4 u, float* f) {
    f[0] = __uint_as_float(u.x);
    f[1] = __uint_as_float(u.y);
    f[2] = __uint_as_float(u.z);
    f[3] = __uint_as_float(u.w);
  }
};

__device__ __forceinline__ int64_t read_slot(int64_t s, int64_t N, int shuffle) {
  if (shuffle) s = (s + N / 2 + 1) % N;  // memory.py:179
  return s < 0 ? 0 : (s >= N ? N - 1 : s);
}

// dw of the R rows of token m into LDS, 512-byte rows (d = 256 fp16 or
// d = 128 fp32), R <= 64: half-waves hold rows 2i and 2i+1 (32 lanes x 16 B
// each); lane partial dots are reduce-scattered across the 32 lanes of a
// half (xor 16, 8, 4, 2, 1), leaving row 2*lane + half in each lane.
template <typename V>
__device__ __forceinline__ void row_dots_512(const V* values, int64_t N, const int32_t* slots, int64_t m, int R,
                                             int shuffle, const float* g, float* dw_lds, int lane) {
  constexpr int VE = RowLoad<V>::kElems;
  const int sub = lane >> 5, col = lane & 31;
  float gv[VE];
#pragma unroll
  for (int e = 0; e < VE; ++e) gv[e] = g[m * (32 * VE) + col * VE + e];
  const int myrow = lane < R ? lane : 0;
  const int64_t myslot = read_slot(slots[m * R + myrow], N, shuffle);
  float part[32];
  const uint4* base = (const uint4*)values;
#pragma unroll
  for (int i0 = 0; i0 < 32; i0 += 8) {
    uint4 buf[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int row = 2 * (i0 + b) + sub;
      const int64_t s = __shfl((int)myslot, row < R ? row : 0);
      buf[b] = base[s * 32 + col];
    }
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      float f[VE];
      RowLoad<V>::unpack(buf[b], f);
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < VE; ++e) acc = fmaf(gv[e], f[e], acc);
      part[i0 + b] = acc;
    }
  }
  // reduce-scatter: after stage s lane keeps the half of the indices whose
  // bit s matches its own
#pragma unroll
  for (int s = 16; s >= 1; s >>= 1) {
    const bool hi = (col & s) != 0;
#pragma unroll
    for (int j = 0; j < s; ++j) {
      const float keep = hi ? part[j + s] : part[j];
      const float send = hi ? part[j] : part[j + s];
      part[j] = keep + __shfl_xor(send, s, 32);
    }
  }
  const int row = 2 * col + sub;
  if (row < R) dw_lds[row] = part[0];
}

// dw of the R rows of token m into LDS, 1 KB rows (d = 256 fp32 or d = 512
// fp16), R <= 64: one row per 16-byte load instruction (64 lanes x 16 B),
// eight rows in flight; lane partial dots are reduce-scattered across the 64
// lanes (xor 32, 16, 8, 4, 2, 1), leaving row `lane` in each lane.
template <typename V>
__device__ __forceinline__ void row_dots_1k(const V* values, int64_t N, const int32_t* slots, int64_t m, int R,
                                            int shuffle, const float* g, float* dw_lds, int lane) {
  constexpr int VE = RowLoad<V>::kElems;
  float gv[VE];
#pragma unroll
  for (int e = 0; e < VE; ++e) gv[e] = g[m * (kWave * VE) + lane * VE + e];
  const int myrow = lane < R ? lane : 0;
  const int64_t myslot = read_slot(slots[m * R + myrow], N, shuffle);
  float part[kWave];
  const uint4* base = (const uint4*)values;
#pragma unroll
  for (int i0 = 0; i0 < kWave; i0 += 8) {
    uint4 buf[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int row = i0 + b;
      const int64_t s = __shfl((int)myslot, row < R ? row : 0);
      buf[b] = base[s * kWave + lane];
    }
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      float f[VE];
      RowLoad<V>::unpack(buf[b], f);
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < VE; ++e) acc = fmaf(gv[e], f[e], acc);
      part[i0 + b] = acc;
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    const bool hi = (lane & s) != 0;
#pragma unroll
    for (int j = 0; j < s; ++j) {
      const float keep = hi ? part[j + s] : part[j];
      const float send = hi ? part[j] : part[j + s];
      part[j] = keep + __shfl_xor(send, s);
    }
  }
  if (lane < R) dw_lds[lane] = part[0];
}

template <typename V>
__device__ __forceinline__ void row_dots_generic(const V* values, int64_t N, int d, const int32_t* slots, int64_t m,
                                                 int R, int shuffle, const float* g, float* dw_lds, int lane) {
  for (int r = lane; r < R; r += kWave) {
    const int64_t s = read_slot(slots[m * R + r], N, shuffle);
    const V* row = values + s * d;
    const float* gr = g + m * d;
    float acc = 0.f;
    for (int j = 0; j < d; ++j) acc = fmaf(gr[j], (float)row[j], acc);
    dw_lds[r] = acc;
  }
}

// MODE 1: 512-byte rows (row_dots_512); 2: 1 KB rows (row_dots_1k); 0: any d.
template <typename V, int MODE>
__global__ __launch_bounds__(kBwdThreads) void route_bwd_kernel(
    const float* __restrict__ g_out, const V* __restrict__ values, int64_t N, int d, const int32_t* __restrict__ slots,
    const float* __restrict__ weights, const int32_t* __restrict__ flat_idx, const float* __restrict__ sub_scores,
    int64_t M, int H, int k, int shuffle, float* __restrict__ d_weights, float* __restrict__ d_sub,
    float* __restrict__ dlogt_part) {
  __shared__ float dw_s[kBwdThreads / kWave][kMaxRows];
  __shared__ float ds_s[kBwdThreads / kWave][kMaxRows];
  __shared__ float w_s[kBwdThreads / kWave][kMaxRows];
  __shared__ int f_s[kBwdThreads / kWave][kMaxRows];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * (kBwdThreads / kWave) + wave;
  if (m >= M) return;  // wave-uniform; no block barrier below
  const int R = H * k;
  float* dw = dw_s[wave];
  float* ds = ds_s[wave];
  // the token's weights and rank pairs, read once (coalesced) for the loops
  // below, which then take them from LDS in the same order
  float* wl = w_s[wave];
  int* fl = f_s[wave];
  for (int r = lane; r < R; r += kWave) {
    wl[r] = weights[m * R + r];
    fl[r] = flat_idx[m * R + r];
  }
  if (MODE == 1)
    row_dots_512<V>(values, N, slots, m, R, shuffle, g_out, dw, lane);
  else if (MODE == 2)
    row_dots_1k<V>(values, N, slots, m, R, shuffle, g_out, dw, lane);
  else
    row_dots_generic<V>(values, N, d, slots, m, R, shuffle, g_out, dw, lane);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  // softmax backward per head (memory.py:178)
  for (int r = lane; r < R; r += kWave) {
    const int h = r / k;
    float s = 0.f;
    for (int j = 0; j < k; ++j) s = fmaf(wl[h * k + j], dw[h * k + j], s);
    const float w = wl[r];
    ds[r] = w * (dw[r] - s);
    if (d_weights != nullptr) d_weights[m * R + r] = dw[r];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  // scatter to the stage-1 ranks, in j order (memory.py:167-175)
  float lt = 0.f;
  for (int o = lane; o < 2 * R; o += kWave) {
    const int h = o / (2 * k);
    const int c = (o / k) & 1;
    const int i = o % k;
    float acc = 0.f;
    for (int j = 0; j < k; ++j) {
      const int f = fl[h * k + j];
      const int rank = c == 0 ? f / k : f % k;
      acc += rank == i ? ds[h * k + j] : 0.f;
    }
    const int64_t so = ((m * H + h) * 2 + c) * k + i;
    d_sub[so] = acc;
    lt = fmaf(acc, sub_scores[so], lt);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) lt += __shfl_xor(lt, off);
  if (lane == 0) dlogt_part[m] = lt;
}

// ---------------------------------------------------------------- queries
// One wave per (m, h, c) row of `half` dims; lane holds dims lane, lane+64.
__global__ __launch_bounds__(kBwdThreads) void queries_bwd_kernel(
    const float* __restrict__ q, const float* __restrict__ q_len, const float* __restrict__ k_hat,
    const int32_t* __restrict__ sub_idx, const float* __restrict__ d_sub, const float* __restrict__ sub_scores,
    const float* __restrict__ extra, const float* __restrict__ dlen_extra, int64_t rows, int HC, int n, int half,
    int k, const float* __restrict__ Tp, float eps, float* __restrict__ dq) {
  const int64_t row = ((int64_t)blockIdx.x * kBwdThreads + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float T = *Tp;
  const int hc = (int)(row % HC);
  const float ql = q_len != nullptr ? q_len[row] : 1.f;
  const float scale = T * ql;
  float dy[2] = {0.f, 0.f};
  float dlen = 0.f;
  // lane i < k holds entry i of the row; entries are broadcast in batches of
  // eight so that sixteen key-row loads per lane are in flight
  const int li = lane < k ? lane : 0;
  const int key_l = sub_idx[row * k + li];
  const float g_l = d_sub[row * k + li];
  const float s_l = q_len != nullptr ? sub_scores[row * k + li] : 0.f;
  if (q_len != nullptr) {
    float t = lane < k ? g_l * (s_l / ql) : 0.f;  // cos * T
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off);
    dlen = t;
  }
  for (int i0 = 0; i0 < k; i0 += 8) {
    float kv[8][2], gs[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int i = i0 + b < k ? i0 + b : 0;
      const int key = __shfl(key_l, i);
      const float g = __shfl(g_l, i);
      const bool ok = i0 + b < k && key >= 0 && key < n;
      gs[b] = ok ? g * scale : 0.f;
      const float* kr = k_hat + ((int64_t)hc * n + (ok ? key : 0)) * half;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int c = lane + kWave * t;
        kv[b][t] = kr[c < half ? c : 0];
      }
    }
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
      for (int t = 0; t < 2; ++t) dy[t] = fmaf(gs[b], kv[b][t], dy[t]);
  }
  if (q_len != nullptr && dlen_extra != nullptr) dlen += dlen_extra[row];
  float x[2], xdy = 0.f, ss = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int c = lane + kWave * t;
    const bool in = c < half;
    x[t] = in ? q[row * half + c] : 0.f;
    if (in && extra != nullptr) dy[t] += extra[row * half + c];
    if (!in) dy[t] = 0.f;
    xdy = fmaf(x[t], dy[t], xdy);
    ss = fmaf(x[t], x[t], ss);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    xdy += __shfl_xor(xdy, off);
    ss += __shfl_xor(ss, off);
  }
  const float s = ss + eps;
  const float r = 1.f / sqrtf(s);
  const float r3 = r * r * r;
  // q_len = sqrt(s) / sqrt(half): d q_len / dx = x / (sqrt(s) sqrt(half))
  const float lenf = q_len != nullptr ? dlen * r / sqrtf((float)half) : 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int c = lane + kWave * t;
    if (c < half) dq[row * half + c] = r * dy[t] - r3 * xdy * x[t] + lenf * x[t];
  }
}

// queries_bwd_kernel for half = 128 with 16-byte rows: a 512-byte k-hat row
// is 32 lanes x 16 B, so one load instruction covers two of the row's
// entries (2b in lanes 0-31, 2b+1 in lanes 32-63) and a row takes a quarter
// of the dword form's load instructions (which are what bounds that form:
// 32 of them per wave, each one address per lane).  Each half-wave sums its
// entries in order, then the two halves are added.
__global__ __launch_bounds__(kBwdThreads) void queries_bwd_128_kernel(
    const float* __restrict__ q, const float* __restrict__ q_len, const float* __restrict__ k_hat,
    const int32_t* __restrict__ sub_idx, const float* __restrict__ d_sub, const float* __restrict__ sub_scores,
    const float* __restrict__ extra, const float* __restrict__ dlen_extra, int64_t rows, int HC, int n, int k,
    const float* __restrict__ Tp, float eps, float* __restrict__ dq) {
  constexpr int HALF = 128;
  const int64_t row = ((int64_t)blockIdx.x * kBwdThreads + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int sub = lane >> 5, col = lane & 31;
  const float T = *Tp;
  const int hc = (int)(row % HC);
  const float ql = q_len != nullptr ? q_len[row] : 1.f;
  const float scale = T * ql;
  const int li = lane < k ? lane : 0;
  const int key_l = sub_idx[row * k + li];
  const float g_l = d_sub[row * k + li];
  float dlen = 0.f;
  if (q_len != nullptr) {
    const float s_l = sub_scores[row * k + li];
    float t = lane < k ? g_l * (s_l / ql) : 0.f;  // cos * T
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off);
    dlen = t;
  }
  const float4* kh = (const float4*)(k_hat + (int64_t)hc * n * HALF);
  float dy[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i0 = 0; i0 < k; i0 += 16) {
    float4 kv[8];
    float gs[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int e = i0 + 2 * b + sub;
      const int i = e < k ? e : 0;
      const int key = __shfl(key_l, i);
      const float g = __shfl(g_l, i);
      const bool ok = e < k && key >= 0 && key < n;
      gs[b] = ok ? g * scale : 0.f;
      kv[b] = kh[(int64_t)(ok ? key : 0) * (HALF / 4) + col];
    }
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      dy[0] = fmaf(gs[b], kv[b].x, dy[0]);
      dy[1] = fmaf(gs[b], kv[b].y, dy[1]);
      dy[2] = fmaf(gs[b], kv[b].z, dy[2]);
      dy[3] = fmaf(gs[b], kv[b].w, dy[3]);
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) dy[t] += __shfl_xor(dy[t], 32);  // both halves now hold dims 4col .. 4col+3
  if (q_len != nullptr && dlen_extra != nullptr) dlen += dlen_extra[row];
  const float4 xv = ((const float4*)(q + row * HALF))[col];
  const float x[4] = {xv.x, xv.y, xv.z, xv.w};
  if (extra != nullptr) {
    const float4 ev = ((const float4*)(extra + row * HALF))[col];
    dy[0] += ev.x;
    dy[1] += ev.y;
    dy[2] += ev.z;
    dy[3] += ev.w;
  }
  float xdy = 0.f, ss = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    xdy = fmaf(x[t], dy[t], xdy);
    ss = fmaf(x[t], x[t], ss);
  }
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) {  // within each half-wave
    xdy += __shfl_xor(xdy, off);
    ss += __shfl_xor(ss, off);
  }
  const float s = ss + eps;
  const float r = 1.f / sqrtf(s);
  const float r3 = r * r * r;
  const float lenf = q_len != nullptr ? dlen * r / sqrtf((float)HALF) : 0.f;
  if (sub == 0) {
    float o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] = r * dy[t] - r3 * xdy * x[t] + lenf * x[t];
    ((float4*)(dq + row * HALF))[col] = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// ------------------------------------------------------------------- keys
__global__ void keys_bwd_prep_kernel(const int32_t* __restrict__ sub_idx, const float* __restrict__ d_sub,
                                     const float* __restrict__ q_len, int64_t P, int HC, int n, int k,
                                     const float* __restrict__ Tp, int32_t* __restrict__ kid,
                                     float* __restrict__ kw) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= P) return;
  const float T = *Tp;
  const int64_t row = p / k;  // (m, h, c)
  const int hc = (int)(row % HC);
  const int key = sub_idx[p];
  const bool ok = key >= 0 && key < n;
  kid[p] = hc * n + (ok ? key : 0);
  kw[p] = ok ? d_sub[p] * T * (q_len != nullptr ? q_len[row] : 1.f) : 0.f;
}

// One wave per key row: dy = merged row (binary search in the ascending
// uniq) + dense extra, then the l2-normalisation backward.
__global__ __launch_bounds__(kBwdThreads) void keys_bwd_kernel(
    const float* __restrict__ keys, const int32_t* __restrict__ uniq, const int32_t* __restrict__ num_unique,
    const float* __restrict__ mrows, const float* __restrict__ extra, int64_t nrows, int half, float eps,
    float* __restrict__ dk) {
  const int64_t j = ((int64_t)blockIdx.x * kBwdThreads + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (j >= nrows) return;
  int lo = 0, hi = *num_unique;  // first u with uniq[u] >= j
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (uniq[mid] < j) lo = mid + 1;
    else hi = mid;
  }
  const bool found = lo < *num_unique && uniq[lo] == j;
  float x[2], dy[2], xdy = 0.f, ss = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int c = lane + kWave * t;
    const bool in = c < half;
    x[t] = in ? keys[j * half + c] : 0.f;
    float v = (in && found) ? mrows[(int64_t)lo * half + c] : 0.f;
    if (in && extra != nullptr) v += extra[j * half + c];
    dy[t] = v;
    xdy = fmaf(x[t], dy[t], xdy);
    ss = fmaf(x[t], x[t], ss);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    xdy += __shfl_xor(xdy, off);
    ss += __shfl_xor(ss, off);
  }
  const float r = 1.f / sqrtf(ss + eps);
  const float r3 = r * r * r;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int c = lane + kWave * t;
    if (c < half) dk[j * half + c] = r * dy[t] - r3 * xdy * x[t];
  }
}

// Fixed-order sum (fp64 accumulation) of x[0, n) plus optional *add.
__global__ __launch_bounds__(1024) void sum_fixed_kernel(const float* __restrict__ x, int64_t n,
                                                         const float* __restrict__ add, float* __restrict__ out) {
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
  if (tid == 0) *out = (float)(part[0] + (add != nullptr ? (double)*add : 0.0));
}

struct KeysLayout {
  size_t kid, kw, uniq, rows, row_sq, nuniq, merge, total, merge_bytes;
  int64_t P, cap;
};

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

static KeysLayout keys_layout(int64_t M, int H, int n, int half, int k) {
  KeysLayout L;
  L.P = M * H * 2 * k;
  const int64_t pool = (int64_t)H * 2 * n;
  L.cap = L.P < pool ? L.P : pool;
  L.merge_bytes = mpl_merge_rows_workspace_bytes(L.P, half, pool);
  size_t o = 0;
  L.kid = o;
  o += al256(L.P * 4);
  L.kw = o;
  o += al256(L.P * 4);
  L.uniq = o;
  o += al256(L.cap * 4);
  L.rows = o;
  o += al256(L.cap * half * 4);
  L.row_sq = o;
  o += al256(L.cap * 4);
  L.nuniq = o;
  o += 256;
  L.merge = o;
  o += al256(L.merge_bytes);
  L.total = o;
  return L;
}

}  // namespace mpl

using namespace mpl;

extern "C" int mpl_lookup_bwd_route(const float* g_out, const void* values, int values_dtype, int64_t N, int d,
                                    const int32_t* slots, const float* weights, const int32_t* flat_idx,
                                    const float* sub_scores, int64_t M, int H, int k, int shuffle_reads,
                                    float* d_weights, float* d_sub, float* dlogt_part, void* stream) {
  clear_error();
  MPL_REQUIRE(N > 0 && d > 0 && M >= 0 && H > 0 && k > 0, MPL_EINVAL, "mpl_lookup_bwd_route: bad sizes");
  MPL_REQUIRE(H * k <= kMaxRows, MPL_EUNSUPPORTED, "mpl_lookup_bwd_route: H*k must be <= %d", kMaxRows);
  MPL_REQUIRE(values_dtype == MPL_F16 || values_dtype == MPL_F32, MPL_EINVAL,
              "mpl_lookup_bwd_route: values_dtype must be MPL_F16 or MPL_F32");
  if (M == 0) return MPL_OK;
  MPL_REQUIRE(g_out && values && slots && weights && flat_idx && sub_scores && d_sub && dlogt_part, MPL_EINVAL,
              "mpl_lookup_bwd_route: null buffer");
  hipStream_t s = (hipStream_t)stream;
  const unsigned blocks = (unsigned)cdiv(M, kBwdThreads / kWave);
  const int esz = values_dtype == MPL_F16 ? 2 : 4;
  const bool vec = H * k <= kWave && ((uintptr_t)values % 16) == 0;
  const int mode = !vec ? 0 : (int64_t)d * esz == 512 ? 1 : (int64_t)d * esz == 1024 ? 2 : 0;
#define MPL_RB(V, F)                                                                                             \
  route_bwd_kernel<V, F><<<blocks, kBwdThreads, 0, s>>>(g_out, (const V*)values, N, d, slots, weights, flat_idx, \
                                                        sub_scores, M, H, k, shuffle_reads, d_weights, d_sub,    \
                                                        dlogt_part)
  if (values_dtype == MPL_F16) {
    if (mode == 1) MPL_RB(_Float16, 1);
    else if (mode == 2) MPL_RB(_Float16, 2);
    else MPL_RB(_Float16, 0);
  } else {
    if (mode == 1) MPL_RB(float, 1);
    else if (mode == 2) MPL_RB(float, 2);
    else MPL_RB(float, 0);
  }
#undef MPL_RB
  return check_launch("mpl_lookup_bwd_route");
}

extern "C" int mpl_lookup_bwd_queries(const float* q, const float* q_len, const float* k_hat, const int32_t* sub_idx,
                                      const float* d_sub, const float* sub_scores, const float* dq_hat_extra,
                                      const float* dlen_extra, int64_t M, int H, int n, int half, int k,
                                      const float* temperature, float* d_queries, void* stream) {
  clear_error();
  MPL_REQUIRE(M >= 0 && H > 0 && n > 0 && k > 0 && half > 0, MPL_EINVAL, "mpl_lookup_bwd_queries: bad sizes");
  MPL_REQUIRE(half <= 2 * kWave, MPL_EUNSUPPORTED, "mpl_lookup_bwd_queries: half must be <= 128");
  MPL_REQUIRE(k <= kWave, MPL_EUNSUPPORTED, "mpl_lookup_bwd_queries: k must be <= %d", kWave);
  if (M == 0) return MPL_OK;
  MPL_REQUIRE(q && k_hat && sub_idx && d_sub && d_queries && temperature && (q_len == nullptr || sub_scores), MPL_EINVAL,
              "mpl_lookup_bwd_queries: null buffer");
  const int64_t rows = M * H * 2;
  const auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const unsigned grid = (unsigned)cdiv(rows, kBwdThreads / kWave);
  if (half == 128 && a16(q) && a16(k_hat) && a16(d_queries) && a16(dq_hat_extra))
    queries_bwd_128_kernel<<<grid, kBwdThreads, 0, (hipStream_t)stream>>>(
        q, q_len, k_hat, sub_idx, d_sub, sub_scores, dq_hat_extra, dlen_extra, rows, 2 * H, n, k, temperature, 1e-6f,
        d_queries);
  else
    queries_bwd_kernel<<<grid, kBwdThreads, 0, (hipStream_t)stream>>>(
        q, q_len, k_hat, sub_idx, d_sub, sub_scores, dq_hat_extra, dlen_extra, rows, 2 * H, n, half, k, temperature,
        1e-6f, d_queries);
  return check_launch("mpl_lookup_bwd_queries");
}

extern "C" size_t mpl_lookup_bwd_keys_workspace_bytes(int64_t M, int H, int n, int half, int k) {
  if (M <= 0 || H <= 0 || n <= 0 || half <= 0 || k <= 0) return 0;
  return keys_layout(M, H, n, half, k).total;
}

extern "C" int mpl_lookup_bwd_keys(const float* sub_keys, const float* q_hat, const float* q_len,
                                   const int32_t* sub_idx, const float* d_sub, const float* dk_hat_extra, int64_t M,
                                   int H, int n, int half, int k, const float* temperature, void* workspace,
                                   size_t workspace_bytes, float* d_sub_keys, void* stream) {
  clear_error();
  MPL_REQUIRE(M >= 0 && H > 0 && n > 0 && k > 0 && half > 0, MPL_EINVAL, "mpl_lookup_bwd_keys: bad sizes");
  MPL_REQUIRE(half <= 2 * kWave, MPL_EUNSUPPORTED, "mpl_lookup_bwd_keys: half must be <= 128");
  MPL_REQUIRE(sub_keys && d_sub_keys, MPL_EINVAL, "mpl_lookup_bwd_keys: null buffer");
  hipStream_t s = (hipStream_t)stream;
  const int64_t nrows = (int64_t)H * 2 * n;
  const unsigned kb = (unsigned)cdiv(nrows, kBwdThreads / kWave);
  if (M == 0) {  // only the dense part (if any) flows back
    // uniq/num_unique are never read when num_unique is 0; use a zero scalar
    static_assert(sizeof(int32_t) == 4, "");
    MPL_REQUIRE(workspace != nullptr && workspace_bytes >= 256, MPL_EWORKSPACE,
                "mpl_lookup_bwd_keys: workspace of 256 bytes needed for M == 0");
    int32_t* zero = (int32_t*)workspace;
    sum_fixed_kernel<<<1, 1024, 0, s>>>(nullptr, 0, nullptr, (float*)zero);  // writes 0.0f == int 0
    keys_bwd_kernel<<<kb, kBwdThreads, 0, s>>>(sub_keys, zero, zero, nullptr, dk_hat_extra, nrows, half, 1e-6f,
                                               d_sub_keys);
    return check_launch("mpl_lookup_bwd_keys");
  }
  MPL_REQUIRE(q_hat && sub_idx && d_sub && temperature, MPL_EINVAL, "mpl_lookup_bwd_keys: null buffer");
  const KeysLayout L = keys_layout(M, H, n, half, k);
  MPL_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, MPL_EWORKSPACE,
              "mpl_lookup_bwd_keys: workspace of %zu bytes needed, %zu given", L.total, workspace_bytes);
  char* ws = (char*)workspace;
  int32_t* kid = (int32_t*)(ws + L.kid);
  float* kw = (float*)(ws + L.kw);
  int32_t* uniq = (int32_t*)(ws + L.uniq);
  float* mrows = (float*)(ws + L.rows);
  float* row_sq = (float*)(ws + L.row_sq);
  int32_t* nuniq = (int32_t*)(ws + L.nuniq);
  keys_bwd_prep_kernel<<<(unsigned)cdiv(L.P, 256), 256, 0, s>>>(sub_idx, d_sub, q_len, L.P, 2 * H, n, k, temperature,
                                                                 kid, kw);
  int rc = check_launch("mpl_lookup_bwd_keys(prep)");
  if (rc) return rc;
  rc = mpl_merge_rows(kid, kw, L.P, k, q_hat, half, nrows, ws + L.merge, L.merge_bytes, uniq, mrows, row_sq, nuniq,
                      0, stream);  // keys_bwd_kernel reads only the rows of keys it finds
  if (rc) return rc;
  keys_bwd_kernel<<<kb, kBwdThreads, 0, s>>>(sub_keys, uniq, nuniq, mrows, dk_hat_extra, nrows, half, 1e-6f,
                                             d_sub_keys);
  return check_launch("mpl_lookup_bwd_keys");
}

extern "C" int mpl_sum(const float* x, int64_t n, const float* add, float* out, void* stream) {
  clear_error();
  MPL_REQUIRE(n >= 0 && out != nullptr && (n == 0 || x != nullptr), MPL_EINVAL, "mpl_sum: bad arguments");
  sum_fixed_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(x, n, add, out);
  return check_launch("mpl_sum");
}
