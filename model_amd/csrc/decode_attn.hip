// One decode step of the backbone's causal self-attention with a key/value
// cache (the decode mode of model.py:29-91's attention: Flax
// MultiHeadDotProductAttention with decode=True, one new token per stream at
// a position shared by every stream, generate.py:31-34).
//
// Per (stream b, head h) one workgroup of 512 threads:
//   q, k, v  <- the fused query/key/value projection row of stream b
//               (qkv [B, 3, heads, hd], biases added; q times `scale`)
//   kt[b, h, :, p] = k,  v_cache[b, h, p, :] = v          (the cache write)
//   s_t = q . k_t for t <= p; w = softmax(s); out[b, h, :] = sum_t w_t v_t
// Positions after p are never read, which is what the reference's mask
// (-inf-like fill before the softmax) leaves of them.  The cache layouts are
// the ones the products read directly: kt [B, heads, hd, max_len] (scores:
// consecutive positions in consecutive lanes), v [B, heads, max_len, hd]
// (weighted sum: consecutive dims in consecutive lanes).  The step's scores
// are kept in LDS (max_len floats), so the kernel reads each cached key and
// value once and writes only the [B, heads * hd] result the output
// projection consumes.  The new position's key and value are used from LDS
// rather than re-read from the cache written in this launch.  The head
// dimension is a template parameter so that the loops over it are unrolled
// and their loads issue back to back.
#include <math.h>

#include "common.h"

namespace mpl {
namespace {

constexpr int kThreads = 512;
constexpr int kMaxLen = 8192;

__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = __shfl_xor(v, off);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  __syncthreads();  // red[] may still be read by the previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kThreads / kWave; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

__device__ __forceinline__ void fma4(float4& acc, float w, const float4& v) {
  acc.x = fmaf(w, v.x, acc.x);
  acc.y = fmaf(w, v.y, acc.y);
  acc.z = fmaf(w, v.z, acc.z);
  acc.w = fmaf(w, v.w, acc.w);
}

template <int HD>
__global__ __launch_bounds__(kThreads) void decode_attention_kernel(const float* __restrict__ qkv, int heads,
                                                                     int max_len, const int64_t* __restrict__ position,
                                                                     float* __restrict__ kt, float* __restrict__ vc,
                                                                     float* __restrict__ out, float scale) {
  constexpr int LP = HD / 4;         // lanes per value row (float4 each)
  constexpr int G = kThreads / LP;   // value-row groups
  constexpr int U = HD <= 64 ? 12 : 4;  // value rows per group loaded at once
  constexpr int DC = HD <= 64 ? HD : 32;  // key dims loaded at once per position
  extern __shared__ float sc[];      // [max_len] scores, then their exponentials
  __shared__ float qs[HD], kn[HD];
  __shared__ float4 vn4[LP];
  __shared__ float4 part[G][LP];
  __shared__ float red[kThreads / kWave];
  const int tid = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / heads, h = bh - b * heads;
  const int64_t pos = *position;
  float* o = out + (size_t)bh * HD;  // out [B, heads, hd] == [B, heads * hd]
  if (pos < 0 || pos >= max_len) {
    // a position outside the cache: nothing is written to the cache and the
    // result is NaN, so the step fails visibly instead of touching memory
    // outside the cache
    if (tid < HD) o[tid] = __builtin_nanf("");
    return;
  }
  const int p = (int)pos;
  const float* row = qkv + (size_t)b * 3 * heads * HD;
  float* ktb = kt + (size_t)bh * HD * max_len;
  float* vb = vc + (size_t)bh * max_len * HD;
  const int g = tid / LP, l4 = tid - g * LP;  // value-row group, float4 of the row
  const float4* vb4 = (const float4*)vb;

  // cache reads that do not depend on the new token go out first: the first
  // DC dims of this thread's first key column (position tid) and the first U
  // value rows of its group (positions g, g + G, ...); positions at or after
  // p read position 0 (in bounds) and are not used
  float kv0[DC];
  {
    const float* col = ktb + (tid < p ? tid : 0);
#pragma unroll
    for (int j = 0; j < DC; ++j) kv0[j] = col[(size_t)j * max_len];
  }
  float4 vv0[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = g + u * G;
    vv0[u] = vb4[(size_t)(t < p ? t : 0) * LP + l4];
  }

  if (tid < HD) {
    const float q = row[h * HD + tid] * scale;
    const float k = row[(heads + h) * HD + tid];
    const float v = row[(2 * heads + h) * HD + tid];
    qs[tid] = q;
    kn[tid] = k;
    ((float*)vn4)[tid] = v;
    ktb[(size_t)tid * max_len + p] = k;
    vb[(size_t)p * HD + tid] = v;
  }
  __syncthreads();

  float mx = -INFINITY;
  for (int t = tid; t <= p; t += kThreads) {
    float s = 0.0f;
    if (t == p) {
#pragma unroll
      for (int d = 0; d < HD; ++d) s = fmaf(qs[d], kn[d], s);
    } else {
      const float* col = ktb + t;
      const bool first = t == tid;
#pragma unroll 1
      for (int d0 = 0; d0 < HD; d0 += DC) {
        float kv[DC];
        if (d0 == 0 && first) {
#pragma unroll
          for (int j = 0; j < DC; ++j) kv[j] = kv0[j];
        } else {
#pragma unroll
          for (int j = 0; j < DC; ++j) kv[j] = col[(size_t)(d0 + j) * max_len];
        }
#pragma unroll
        for (int j = 0; j < DC; ++j) s = fmaf(qs[d0 + j], kv[j], s);
      }
    }
    sc[t] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_reduce(mx, red, true);
  float sum = 0.0f;
  for (int t = tid; t <= p; t += kThreads) {
    const float e = expf(sc[t] - mx);
    sc[t] = e;
    sum += e;
  }
  sum = block_reduce(sum, red, false);  // its barriers also publish sc[]

  // weighted sum of the values: group g takes positions t = g, g + G, ...
  // (the first U from the registers loaded at the start, then U per step,
  // loads first); lane l4 of a group owns dims 4 l4 .. 4 l4 + 3; position p
  // itself comes from LDS
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = g + u * G;
    if (t < p) fma4(acc, sc[t], vv0[u]);
  }
  int t = g + U * G;
  for (; t < p; t += U * G) {
    float4 vv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int tu = t + u * G;
      vv[u] = vb4[(size_t)(tu < p ? tu : 0) * LP + l4];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (t + u * G < p) fma4(acc, sc[t + u * G], vv[u]);
  }
  if (p % G == g) fma4(acc, sc[p], vn4[l4]);  // the group whose sequence reaches p
  part[g][l4] = acc;
  __syncthreads();
  if (tid < HD) {
    const int q4 = tid / 4, e = tid % 4;
    float a = 0.0f;
    for (int j = 0; j < G; ++j) a += ((const float*)&part[j][q4])[e];
    o[tid] = a / sum;
  }
}

}  // namespace
}  // namespace mpl

using namespace mpl;

extern "C" int mpl_decode_attention(const float* qkv, int64_t batch, int heads, int head_dim, int max_len,
                                    const int64_t* position, float* k_cache_t, float* v_cache, float* out,
                                    float scale, void* stream) {
  clear_error();
  MPL_REQUIRE(batch >= 0 && heads >= 1, MPL_EINVAL, "mpl_decode_attention: bad batch=%lld heads=%d",
              (long long)batch, heads);
  MPL_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256, MPL_EINVAL,
              "mpl_decode_attention: head_dim=%d must be 16, 32, 64, 128 or 256", head_dim);
  MPL_REQUIRE(max_len >= 1 && max_len <= kMaxLen, MPL_EINVAL, "mpl_decode_attention: max_len=%d outside [1, %d]",
              max_len, kMaxLen);
  MPL_REQUIRE(batch * heads <= INT32_MAX, MPL_EINVAL, "mpl_decode_attention: batch * heads too large");
  if (batch == 0) return MPL_OK;
  MPL_REQUIRE(qkv && position && k_cache_t && v_cache && out, MPL_EINVAL, "mpl_decode_attention: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const unsigned grid = (unsigned)(batch * heads);
  const size_t lds = (size_t)max_len * sizeof(float);
#define MPL_DECODE_ATTN(HD)                                                                                      \
  decode_attention_kernel<HD><<<grid, kThreads, lds, s>>>(qkv, heads, max_len, position, k_cache_t, v_cache, out, \
                                                          scale)
  switch (head_dim) {
    case 16: MPL_DECODE_ATTN(16); break;
    case 32: MPL_DECODE_ATTN(32); break;
    case 64: MPL_DECODE_ATTN(64); break;
    case 128: MPL_DECODE_ATTN(128); break;
    default: MPL_DECODE_ATTN(256); break;
  }
#undef MPL_DECODE_ATTN
  return check_launch("mpl_decode_attention");
}
