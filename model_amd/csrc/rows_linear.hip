// Dense layers of the backbone for a few rows at a time (one decode step:
// one row per stream), with what surrounds them in model.py:29-127 fused in:
//
//   a   = x                          (rows [R, K] fp32)
//   a   = LayerNorm(a) * g + beta    if ln_scale (flax LayerNorm: mean and
//                                    biased variance over K, eps inside the
//                                    square root)
//   a   = a * x_mul                  if x_mul (the gated memory read
//                                    mem * gate before mem_out)
//   out = act(a . W + bias) + residual        act: none, gelu (tanh form), silu
//
// W is [K, N] (a Dense kernel) or [N, K] (the embedding table read by
// embed.attend).  Library GEMMs pick tiles for large matrices; here the
// products are R x K x N with R = a few dozen rows (one per stream), which
// leaves a 16-row tile per workgroup and makes the number of dependent
// memory round trips of a thread the cost.  So K is split over all 512
// threads of the workgroup that owns a 16 x 16 output tile: lane (ks, cp) of
// wave w takes the float4 columns j = 8w + ks, +64, +128, ... of K for the
// output columns 2cp and 2cp + 1 and all 16 rows (32 accumulators), and
// issues the row and weight loads of two such columns before the first FMA
// (one column per thread at K = 256, two batches at K = 1,024).  The 8
// K-slices of a wave are then added by a shuffle reduce-scatter (xor 32, 16,
// 8: each step halves the values a lane holds), the 8 waves' partial tiles
// through LDS in a fixed order, so results are deterministic.  LayerNorm
// statistics of the tile's rows are computed first (two passes over each
// row, mean then centred variance, from registers) while the first weights
// are in flight, and the normalisation is applied to the operand as it is
// loaded.
#include <math.h>

#include "common.h"
#include "topk.h"

namespace mpl {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kTR = 16;                // rows per tile
constexpr int kTN = 16;                // columns per tile
constexpr int kSlices = kThreads / 8;  // K-slices per workgroup

struct LinearArgs {
  const float* x;
  const float* x_mul;
  const float* ln_scale;
  const float* ln_bias;
  const float* w;
  const float* bias;
  const float* residual;
  float* out;
  int64_t rows;
  int K, N, act;
  float eps;
  // two layers of one input as one product: output columns [n1, N) go to
  // out2 [rows, N - n1] with activation act2 (n1 == N: one layer)
  float* out2;
  int n1, act2;
};

__device__ __forceinline__ float activate(float v, int act) {
  if (act == MPL_ACT_GELU_TANH) {
    // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
    const float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    return 0.5f * v * (1.0f + tanhf(inner));
  }
  if (act == MPL_ACT_SILU) return v / (1.0f + expf(-v));
  return v;
}

// One reduce-scatter step over lanes l and l ^ OFF: of the C values a lane
// holds, the lane with bit OFF set keeps (and receives the partner's copy of)
// the upper half, the other the lower half.
template <int C, int OFF>
__device__ __forceinline__ void scatter_step(float* v, int lane) {
  const bool up = (lane & OFF) != 0;
#pragma unroll
  for (int q = 0; q < C / 2; ++q) {
    const float send = up ? v[q] : v[q + C / 2];
    const float keep = up ? v[q + C / 2] : v[q];
    v[q] = keep + __shfl_xor(send, OFF);
  }
}

__device__ __forceinline__ void fma4(float& acc, const float4& v, const float4& w) {
  acc = fmaf(v.x, w.x, acc);
  acc = fmaf(v.y, w.y, acc);
  acc = fmaf(v.z, w.z, acc);
  acc = fmaf(v.w, w.w, acc);
}

// U: K columns per thread whose loads are in flight together (1 when a
// thread has a single column, K <= 4 * kSlices).  TR: rows per tile, 16, or
// 4 for narrow products (N = 256 at 64 rows: 256 workgroups instead of 64);
// the per-element summation order is the same for both.  (8-row tiles for
// the layer-normalised decode products measured slower: 0.245 against
// 0.235 ms per generation step.)
template <int LAYOUT, bool LN, bool MUL, int U, int TR = kTR>
__global__ __launch_bounds__(kThreads) void rows_linear_kernel(LinearArgs a) {
  static_assert(TR == 16 || (TR == 4 && !LN), "16-row tiles, or 4-row tiles without the layer norm");
  __shared__ float red[kWaves][TR * kTN];
  __shared__ float s_mean[TR], s_rstd[TR];
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int64_t r0 = (int64_t)blockIdx.y * TR;
  const int n0 = blockIdx.x * kTN;
  const int K = a.K, K4 = K / 4;
  const int nrows = (int)min<int64_t>(TR, a.rows - r0);  // valid rows of this tile

  // operands that do not depend on the row statistics are requested first:
  // the epilogue's bias and residual element of this thread (threads below
  // TR * kTN) and the weights of its first K columns
  const int erow = tid / kTN, ecol = tid % kTN;
  const int en = n0 + ecol;
  const bool eval = tid < TR * kTN && erow < nrows && en < a.N;
  const int64_t eat = (r0 + erow) * a.N + en;
  const float ebias = (eval && a.bias) ? a.bias[en] : 0.0f;
  const float eres = (eval && a.residual) ? a.residual[eat] : 0.0f;

  const int cp = lane % 8, ks = lane / 8;
  const int c0 = n0 + 2 * cp;
  const bool cval = c0 < a.N, cval1 = c0 + 1 < a.N;
  const bool pairs = (a.N & 1) == 0;  // [K, N] rows hold aligned column pairs
  const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  auto load_w = [&](int k, float4& w0, float4& w1) {
    w0 = zero;
    w1 = zero;
    if (LAYOUT == MPL_W_OUT_IN) {
      if (cval) w0 = *(const float4*)(a.w + (int64_t)c0 * K + k);
      if (cval1) w1 = *(const float4*)(a.w + (int64_t)(c0 + 1) * K + k);
    } else if (cval1 && pairs) {
      const float2 u0 = *(const float2*)(a.w + (int64_t)k * a.N + c0);
      const float2 u1 = *(const float2*)(a.w + (int64_t)(k + 1) * a.N + c0);
      const float2 u2 = *(const float2*)(a.w + (int64_t)(k + 2) * a.N + c0);
      const float2 u3 = *(const float2*)(a.w + (int64_t)(k + 3) * a.N + c0);
      w0 = make_float4(u0.x, u1.x, u2.x, u3.x);
      w1 = make_float4(u0.y, u1.y, u2.y, u3.y);
    } else if (cval) {
      const float* wc = a.w + (int64_t)k * a.N + c0;
      w0 = make_float4(wc[0], wc[a.N], wc[2 * (int64_t)a.N], wc[3 * (int64_t)a.N]);
      if (cval1) w1 = make_float4(wc[1], wc[a.N + 1], wc[2 * (int64_t)a.N + 1], wc[3 * (int64_t)a.N + 1]);
    }
  };
  const int j0 = wave * 8 + ks;
  // the columns of a batch: j, j + kSlices, ..., clamped to the last valid
  // column (their loads stay in bounds; a clamped column is not accumulated)
  float4 w0[U], w1[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = min(j0 + u * kSlices, K4 - 1);
    load_w(4 * j, w0[u], w1[u]);
  }

  // the first batch of rows (and x_mul rows, LayerNorm scale and shift) is
  // requested before the row statistics too: the loads do not depend on them
  const float* xt = a.x + r0 * K;
  const float* mt = MUL ? a.x_mul + r0 * K : nullptr;
  float4 xv[U][TR];
  float4 mv[LN && MUL ? U : 1][TR];  // x_mul rows, applied after the normalisation
  float4 g[U], be[U];
  auto load_batch = [&](int jb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = 4 * min(jb + u * kSlices, K4 - 1);
      g[u] = LN ? *(const float4*)(a.ln_scale + k) : zero;
      be[u] = LN ? *(const float4*)(a.ln_bias + k) : zero;
#pragma unroll
      for (int i = 0; i < TR; ++i) {
        // rows past the end read row 0 (in bounds) and are never stored
        const int64_t off = (int64_t)(i < nrows ? i : 0) * K + k;
        float4 v = *(const float4*)(xt + off);
        if (MUL) {
          const float4 m = *(const float4*)(mt + off);
          if (LN) {
            mv[LN && MUL ? u : 0][i] = m;
          } else {
            v.x *= m.x;
            v.y *= m.y;
            v.z *= m.z;
            v.w *= m.w;
          }
        }
        xv[u][i] = v;
      }
    }
  };
  load_batch(j0);

  if (LN) {
    // 32 threads per row (consecutive lanes); a thread's part of the row is
    // kept in registers between the two passes when it has at most kHold
    // float4s (K <= 512), and read again otherwise
    constexpr int TPR = kThreads / TR;
    constexpr int kHold = 4;
    const int row = tid / TPR, part = tid % TPR;
    const float4* xr = (const float4*)(a.x + (r0 + (row < nrows ? row : 0)) * K);
    const bool hold = K4 <= kHold * TPR;
    float4 hv[kHold];
    float s = 0.0f;
    if (row < nrows) {
      if (hold) {
        // clamped loads, zeroed after: a select of the load's address would
        // turn them into flat loads of a private zero
#pragma unroll
        for (int h = 0; h < kHold; ++h) {
          const int j = part + h * TPR;
          hv[h] = xr[j < K4 ? j : K4 - 1];
        }
#pragma unroll
        for (int h = 0; h < kHold; ++h)
          if (part + h * TPR >= K4) hv[h] = zero;
#pragma unroll
        for (int h = 0; h < kHold; ++h) s += (hv[h].x + hv[h].y) + (hv[h].z + hv[h].w);
      } else {
        for (int j = part; j < K4; j += TPR) {
          const float4 v = xr[j];
          s += (v.x + v.y) + (v.z + v.w);
        }
      }
    }
    for (int off = TPR / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, TPR);
    const float mean = s / (float)K;
    float q = 0.0f;
    if (row < nrows) {
      if (hold) {
#pragma unroll
        for (int h = 0; h < kHold; ++h) {
          if (part + h * TPR < K4) {
            const float d0 = hv[h].x - mean, d1 = hv[h].y - mean, d2 = hv[h].z - mean, d3 = hv[h].w - mean;
            q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
          }
        }
      } else {
        for (int j = part; j < K4; j += TPR) {
          const float4 v = xr[j];
          const float d0 = v.x - mean, d1 = v.y - mean, d2 = v.z - mean, d3 = v.w - mean;
          q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
      }
    }
    for (int off = TPR / 2; off >= 1; off >>= 1) q += __shfl_xor(q, off, TPR);
    if (part == 0) {
      s_mean[row] = mean;
      s_rstd[row] = rsqrtf(q / (float)K + a.eps);
    }
    __syncthreads();
  }

  float acc[2 * TR];  // acc[2 i + c]: row i, column c0 + c
#pragma unroll
  for (int e = 0; e < 2 * TR; ++e) acc[e] = 0.0f;

  for (int jb = j0; jb < K4; jb += U * kSlices) {
    if (jb != j0) load_batch(jb);  // the first batch was requested before the statistics
    // the next batch's weights go out before this batch's arithmetic
    float4 nw0[U], nw1[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = min(jb + (U + u) * kSlices, K4 - 1);
      if (jb + U * kSlices < K4) load_w(4 * j, nw0[u], nw1[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (jb + u * kSlices >= K4) break;  // a clamped column of the last batch
#pragma unroll
      for (int i = 0; i < TR; ++i) {
        float4 v = xv[u][i];
        if (LN) {
          const float mean = s_mean[i], rstd = s_rstd[i];
          v.x = (v.x - mean) * rstd * g[u].x + be[u].x;
          v.y = (v.y - mean) * rstd * g[u].y + be[u].y;
          v.z = (v.z - mean) * rstd * g[u].z + be[u].z;
          v.w = (v.w - mean) * rstd * g[u].w + be[u].w;
          if (MUL) {
            const float4 m = mv[LN && MUL ? u : 0][i];
            v.x *= m.x;
            v.y *= m.y;
            v.z *= m.z;
            v.w *= m.w;
          }
        }
        fma4(acc[2 * i], v, w0[u]);
        fma4(acc[2 * i + 1], v, w1[u]);
      }
    }
    if (jb + U * kSlices < K4) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        w0[u] = nw0[u];
        w1[u] = nw1[u];
      }
    }
  }

  // the wave's 8 K-slices (lane bits 3..5): afterwards lane (ks, cp) holds
  // the sums of acc[e], e = (TR / 4) ks + q, q < TR / 4, i.e. row e / 2,
  // column 2 cp + e % 2 (every element's sum is ((s0 + s4) + (s2 + s6)) +
  // ((s1 + s5) + (s3 + s7)) over the slices, whatever TR is)
  scatter_step<2 * TR, 32>(acc, lane);
  scatter_step<TR, 16>(acc, lane);
  scatter_step<TR / 2, 8>(acc, lane);
#pragma unroll
  for (int q = 0; q < TR / 4; ++q) {
    const int e = (TR / 4) * ks + q;
    red[wave][(e >> 1) * kTN + 2 * cp + (e & 1)] = acc[q];
  }
  __syncthreads();
  if (eval) {
    const int o = tid;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v += red[w][o];
    if (en < a.n1) {
      v = activate(v + ebias, a.act);
      a.out[(r0 + erow) * a.n1 + en] = v + eres;
    } else {
      v = activate(v + ebias, a.act2);
      a.out2[(r0 + erow) * (a.N - a.n1) + (en - a.n1)] = v + eres;
    }
  }
}

template <int LAYOUT>
void launch_rows_linear(const LinearArgs& a, bool ln, bool mul, hipStream_t s) {
  // narrow products without the layer norm (N = 256 at 64 rows: the
  // attention and feed-forward outputs, the memory read's output) take
  // 4-row tiles, all their K columns in one batch of loads
  if (!ln && cdiv(a.N, kTN) * cdiv(a.rows, kTR) < 128 && a.K <= 1024) {
    const dim3 g4((unsigned)cdiv(a.N, kTN), (unsigned)cdiv(a.rows, 4));
    if (mul)
      rows_linear_kernel<LAYOUT, false, true, 1, 4><<<g4, kThreads, 0, s>>>(a);
    else if (a.K / 4 > kSlices)
      rows_linear_kernel<LAYOUT, false, false, 4, 4><<<g4, kThreads, 0, s>>>(a);
    else
      rows_linear_kernel<LAYOUT, false, false, 1, 4><<<g4, kThreads, 0, s>>>(a);
    return;
  }
  const dim3 grid((unsigned)cdiv(a.N, kTN), (unsigned)cdiv(a.rows, kTR));
  // two columns in flight only for the plain product with more than one
  // column per thread (the feed-forward output, K = 1,024): with a layer
  // norm or x_mul the second batch of row registers would spill
  if (ln && mul)
    rows_linear_kernel<LAYOUT, true, true, 1><<<grid, kThreads, 0, s>>>(a);
  else if (ln)
    rows_linear_kernel<LAYOUT, true, false, 1><<<grid, kThreads, 0, s>>>(a);
  else if (mul)
    rows_linear_kernel<LAYOUT, false, true, 1><<<grid, kThreads, 0, s>>>(a);
  else if (a.K / 4 > kSlices)
    rows_linear_kernel<LAYOUT, false, false, 2><<<grid, kThreads, 0, s>>>(a);
  else
    rows_linear_kernel<LAYOUT, false, false, 1><<<grid, kThreads, 0, s>>>(a);
}

// The output layer of a decode step (model.py:125-126): logits [rows, V] =
// LayerNorm(x) . emb^T (embed.attend of ln_final), rows <= 64, d <= 256 with
// d % 4 == 0.  A workgroup owns 64 vocabulary rows.  Wave w loads rows
// w, w + 4, ... of x and of the tile's embedding rows, lane c the float4 at
// column 4c, all 32 loads before any use; each x row's LayerNorm statistics
// (mean, then the centred variance, rsqrt(var + eps)) are wave reductions of
// the registers, and the normalised rows go to LDS beside the embedding rows.
// Each wave then forms one 32 x 32 block of the tile with fp32 MFMAs
// (v_mfma_f32_32x32x2_f32: lane l gives element (l % 32, k) of A = x rows and
// B = embedding rows and holds logits[8 (r/4) + 4 (l/32) + r%4][l % 32] in
// r).  The K order is permuted so that one 16-byte LDS read feeds four
// MFMAs: over an 8-column group, MFMA i of the group takes columns i and
// i + 4 (lanes 0-31 and 32-63), and even and odd MFMAs go to two accumulator
// chains.  The LDS pitch (d + 4 floats) keeps rows 16-byte aligned, and the
// 8 lanes of a 16-byte read phase cover all banks.
constexpr int kVT = 256;       // threads (4 waves: 2 x 2 blocks)
constexpr int kVR = 64;        // x rows (streams) per tile
constexpr int kVV = 64;        // vocabulary rows per tile
constexpr int kVP4 = 65;       // LDS pitch in float4 (d <= 256, plus one)

// v[i] = the sum of v[i] over the wave, in every lane, for N values at
// once (exchanges on DPP and permlane, no LDS).
template <int N>
__device__ __forceinline__ void wave_allsum(float (&v)[N], int lane) {
#define MPL_XSUM(S)                                                                        \
  _Pragma("unroll") for (int i = 0; i < N; ++i) v[i] += __uint_as_float(w64::xr<S>(__float_as_uint(v[i]), lane));
  MPL_XSUM(32) MPL_XSUM(16) MPL_XSUM(8) MPL_XSUM(4) MPL_XSUM(2) MPL_XSUM(1)
#undef MPL_XSUM
}

__global__ __launch_bounds__(kVT) void vocab_logits_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ ln_scale,
                                                           const float* __restrict__ ln_bias, float eps,
                                                           const float* __restrict__ emb, int rows, int d,
                                                           int64_t V, float* __restrict__ out) {
  __shared__ float4 sX[kVR * kVP4];
  __shared__ float4 sE[kVV * kVP4];
  constexpr int kPer = kVR / (kVT / 64);  // rows per wave
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t v0 = (int64_t)blockIdx.x * kVV;
  const int d4 = d >> 2;
  const bool colok = lane < d4;  // lanes past the row end store zeros
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  // every load is issued unconditionally at a clamped (in-bounds) address
  // and zeroed after, so that all 34 go out back to back
  const int c4 = 4 * (colok ? lane : d4 - 1);
  float4 ev[kPer], xv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int r = 4 * i + wave;
    const int64_t v = v0 + r;
    ev[i] = *(const float4*)(emb + (v < V ? v : V - 1) * d + c4);
    xv[i] = *(const float4*)(x + (int64_t)(r < rows ? r : rows - 1) * d + c4);
  }
  float4 g4 = *(const float4*)(ln_scale + c4);
  float4 b4 = *(const float4*)(ln_bias + c4);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int r = 4 * i + wave;
    if (!colok || v0 + r >= V) ev[i] = z4;
    if (!colok || r >= rows) xv[i] = z4;
  }
  if (!colok) g4 = b4 = z4;
#pragma unroll
  for (int i = 0; i < kPer; ++i) sE[(4 * i + wave) * kVP4 + lane] = ev[i];
  const float inv_d = 1.f / (float)d;
  float mean[kPer], var[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) mean[i] = (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
  wave_allsum<kPer>(mean, lane);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    mean[i] *= inv_d;
    if (colok) {
      xv[i].x -= mean[i]; xv[i].y -= mean[i]; xv[i].z -= mean[i]; xv[i].w -= mean[i];
    }
    var[i] = (xv[i].x * xv[i].x + xv[i].y * xv[i].y) + (xv[i].z * xv[i].z + xv[i].w * xv[i].w);
  }
  wave_allsum<kPer>(var, lane);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int r = 4 * i + wave;
    const float rs = rsqrtf(var[i] * inv_d + eps);
    float4 y = z4;  // rows past `rows` and columns past d stay zero
    if (colok && r < rows) {
      y.x = xv[i].x * rs * g4.x + b4.x;
      y.y = xv[i].y * rs * g4.y + b4.y;
      y.z = xv[i].z * rs * g4.z + b4.z;
      y.w = xv[i].w * rs * g4.w + b4.w;
    }
    sX[r * kVP4 + lane] = y;
  }
  __syncthreads();
  const int li = lane & 31, lk = lane >> 5;
  const int tb = wave >> 1, vb = wave & 1;
  const float4* pa = sX + (32 * tb + li) * kVP4 + lk;
  const float4* pb = sE + (32 * vb + li) * kVP4 + lk;
  f32x16 acc0 = f32x16{}, acc1 = f32x16{};
  // all 256 columns, unrolled so that LDS reads run ahead of the MFMAs:
  // columns past d hold the zeros stored above
#pragma unroll
  for (int gi = 0; gi < 32; ++gi) {
    const float4 av = pa[2 * gi], bv = pb[2 * gi];
    acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc1, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc1, 0, 0, 0);
  }
  const int64_t v = v0 + 32 * vb + li;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 32 * tb + 8 * (r >> 2) + 4 * lk + (r & 3);
    if (row < rows && v < V) out[(int64_t)row * V + v] = acc0[r] + acc1[r];
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace mpl

using namespace mpl;

extern "C" int mpl_rows_linear(const float* x, const float* x_mul, const float* ln_scale, const float* ln_bias,
                               float ln_eps, const float* weight, int weight_layout, const float* bias, int activation,
                               const float* residual, int64_t rows, int K, int N, float* out, void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && K >= 4 && K % 4 == 0 && N >= 1, MPL_EINVAL,
              "mpl_rows_linear: rows=%lld K=%d N=%d (K must be a positive multiple of 4, N positive)",
              (long long)rows, K, N);
  MPL_REQUIRE(weight_layout == MPL_W_IN_OUT || weight_layout == MPL_W_OUT_IN, MPL_EINVAL,
              "mpl_rows_linear: bad weight_layout %d", weight_layout);
  MPL_REQUIRE(activation == MPL_ACT_NONE || activation == MPL_ACT_GELU_TANH || activation == MPL_ACT_SILU,
              MPL_EINVAL, "mpl_rows_linear: bad activation %d", activation);
  MPL_REQUIRE((ln_scale == nullptr) == (ln_bias == nullptr), MPL_EINVAL,
              "mpl_rows_linear: ln_scale and ln_bias go together");
  MPL_REQUIRE(rows <= (int64_t)65535 * 16, MPL_EINVAL, "mpl_rows_linear: rows=%lld above %d", (long long)rows,
              65535 * 16);
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(x && weight && out, MPL_EINVAL, "mpl_rows_linear: null x, weight or out");
  MPL_REQUIRE(aligned16(x) && aligned16(weight) && aligned16(x_mul) && aligned16(ln_scale) && aligned16(ln_bias),
              MPL_EINVAL, "mpl_rows_linear: x, x_mul, weight, ln_scale and ln_bias must be 16-byte aligned");
  MPL_REQUIRE(out != x && out != x_mul, MPL_EINVAL, "mpl_rows_linear: out may alias residual only");
  LinearArgs a{x, x_mul, ln_scale, ln_bias, weight, bias, residual, out, rows, K, N, activation, ln_eps,
               nullptr, N, activation};
  hipStream_t s = (hipStream_t)stream;
  const bool ln = ln_scale != nullptr, mul = x_mul != nullptr;
  if (weight_layout == MPL_W_OUT_IN)
    launch_rows_linear<MPL_W_OUT_IN>(a, ln, mul, s);
  else
    launch_rows_linear<MPL_W_IN_OUT>(a, ln, mul, s);
  return check_launch("mpl_rows_linear");
}

extern "C" int mpl_vocab_logits(const float* x, const float* ln_scale, const float* ln_bias, float ln_eps,
                                const float* emb, int64_t rows, int d, int64_t V, float* logits, void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && d > 0 && V > 0, MPL_EINVAL, "mpl_vocab_logits: bad sizes");
  MPL_REQUIRE(rows <= kVR && d <= 256 && d % 4 == 0, MPL_EUNSUPPORTED,
              "mpl_vocab_logits: needs rows <= %d and d a multiple of 4 up to 256 (rows %lld, d %d)", kVR,
              (long long)rows, d);
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(x && ln_scale && ln_bias && emb && logits, MPL_EINVAL, "mpl_vocab_logits: null buffer");
  MPL_REQUIRE(aligned16(x) && aligned16(ln_scale) && aligned16(ln_bias) && aligned16(emb), MPL_EINVAL,
              "mpl_vocab_logits: x, ln_scale, ln_bias and emb must be 16-byte aligned");
  const int64_t tiles = (V + kVV - 1) / kVV;
  MPL_REQUIRE(tiles < ((int64_t)1 << 31), MPL_EUNSUPPORTED, "mpl_vocab_logits: vocabulary too large");
  vocab_logits_kernel<<<(unsigned)tiles, kVT, 0, (hipStream_t)stream>>>(x, ln_scale, ln_bias, ln_eps, emb,
                                                                      (int)rows, d, V, logits);
  return check_launch("mpl_vocab_logits");
}

extern "C" int mpl_rows_linear_pair(const float* x, const float* ln_scale, const float* ln_bias, float ln_eps,
                                    const float* weight, const float* bias, int activation1, int activation2,
                                    int64_t rows, int K, int N1, int N2, float* out1, float* out2, void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && K >= 4 && K % 4 == 0 && N1 >= 1 && N2 >= 1, MPL_EINVAL,
              "mpl_rows_linear_pair: rows=%lld K=%d N1=%d N2=%d (K a positive multiple of 4, N1 and N2 positive)",
              (long long)rows, K, N1, N2);
  auto act_ok = [](int act) { return act == MPL_ACT_NONE || act == MPL_ACT_GELU_TANH || act == MPL_ACT_SILU; };
  MPL_REQUIRE(act_ok(activation1) && act_ok(activation2), MPL_EINVAL, "mpl_rows_linear_pair: bad activation %d / %d",
              activation1, activation2);
  MPL_REQUIRE((ln_scale == nullptr) == (ln_bias == nullptr), MPL_EINVAL,
              "mpl_rows_linear_pair: ln_scale and ln_bias go together");
  MPL_REQUIRE(rows <= (int64_t)65535 * 16, MPL_EINVAL, "mpl_rows_linear_pair: rows=%lld above %d", (long long)rows,
              65535 * 16);
  MPL_REQUIRE((int64_t)N1 + N2 < ((int64_t)1 << 31), MPL_EINVAL, "mpl_rows_linear_pair: N1 + N2 too large");
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(x && weight && out1 && out2, MPL_EINVAL, "mpl_rows_linear_pair: null x, weight, out1 or out2");
  MPL_REQUIRE(aligned16(x) && aligned16(weight) && aligned16(ln_scale) && aligned16(ln_bias), MPL_EINVAL,
              "mpl_rows_linear_pair: x, weight, ln_scale and ln_bias must be 16-byte aligned");
  MPL_REQUIRE(out1 != x && out2 != x && out1 != out2, MPL_EINVAL, "mpl_rows_linear_pair: outputs may not alias");
  LinearArgs a{x, nullptr, ln_scale, ln_bias, weight, bias, nullptr, out1, rows, K, N1 + N2, activation1, ln_eps,
               out2, N1, activation2};
  launch_rows_linear<MPL_W_IN_OUT>(a, ln_scale != nullptr, false, (hipStream_t)stream);
  return check_launch("mpl_rows_linear_pair");
}
