// The greedy generator's per-step token work on the GPU (generate.py:44-61:
// feed the next prompt token while the prompt lasts, then take the argmax of
// the step's logits and append it to the output), so that a whole greedy
// decode step, model and token choice, is one HIP graph replay with no host
// work in between.
//
// One workgroup of 256 threads per stream b reads p = *position, and:
//   next = prompt[b, p + 1]               if p + 1 < prompt_len
//   next = argmax_v logits[b, v]          otherwise (the first maximal index,
//                                         as torch.argmax; NaN counts as the
//                                         maximum, also as torch.argmax)
//   token[b] = next;  out[b, p + 1 - prompt_len] = next  (generated tokens)
// The last workgroup to finish (an atomic count, reset by that workgroup)
// advances *position to p + 1, after every workgroup has read p.
//
// The step's input rows (embedding plus position embedding) are one launch
// too: decode_embed_kernel below.
#include <math.h>

#include "common.h"

namespace mpl {
namespace {

constexpr int kTokThreads = 256;

// (value, index) order of torch.argmax: NaN above everything, then larger
// values, then, among equal values, the smaller index.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  const bool vn = isnan(v), bn = isnan(bv);
  if (vn != bn) return vn;
  if (!vn && v != bv) return v > bv;
  return i < bi;
}

__global__ __launch_bounds__(kTokThreads) void next_token_kernel(const float* __restrict__ logits, int64_t vocab,
                                                                 const int64_t* __restrict__ prompt,
                                                                 int64_t prompt_stride,
                                                                 const int64_t* __restrict__ prompt_len,
                                                                 int64_t* __restrict__ position,
                                                                 int64_t* __restrict__ token,
                                                                 int64_t* __restrict__ out, int64_t out_stride,
                                                                 int64_t out_cap, uint32_t* __restrict__ done,
                                                                 const float* __restrict__ emb, int64_t emb_rows,
                                                                 const float* __restrict__ pos_emb,
                                                                 int64_t max_pos, int d4,
                                                                 float* __restrict__ x_next) {
  __shared__ float rv[kTokThreads / kWave];
  __shared__ int ri[kTokThreads / kWave];
  __shared__ int64_t sp[2];
  __shared__ int last;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  // thread 0 reads the position once for the workgroup: after this barrier
  // no wave of the workgroup reads it again, so the workgroup's count below
  // comes after its read, and the last workgroup may advance it
  if (tid == 0) {
    sp[0] = *position;
    sp[1] = *prompt_len;
  }
  __syncthreads();
  const int64_t p = sp[0];
  const int64_t P = sp[1];
  int64_t next;
  if (p + 1 >= 0 && p + 1 < P) {
    next = prompt[b * prompt_stride + p + 1];  // workgroup-uniform branch
  } else {
    const float* row = logits + b * vocab;
    const int V = (int)vocab;
    float bv = -INFINITY;
    int bi = V;  // above every index: any element beats it
    // 16-byte loads, kBatch per thread issued before any is compared (the
    // order of the comparisons does not matter: `better` is a total order)
    constexpr int kBatch = 16;
    const bool vec = (V & 3) == 0 && ((uintptr_t)row & 15) == 0;  // workgroup-uniform
    const int nv = vec ? V / 4 : 0;
    const float4* row4 = (const float4*)row;
    for (int base = 0; base < nv; base += kBatch * kTokThreads) {
      float4 x[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = base + u * kTokThreads + tid;
        x[u] = row4[i < nv ? i : 0];
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = base + u * kTokThreads + tid;
        if (i < nv) {
          const float e[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (better(e[j], 4 * i + j, bv, bi)) {
              bv = e[j];
              bi = 4 * i + j;
            }
        }
      }
    }
    for (int v = 4 * nv + tid; v < V; v += kTokThreads) {  // rows that are not whole 16-byte vectors
      const float x = row[v];
      if (better(x, v, bv, bi)) {
        bv = x;
        bi = v;
      }
    }
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (tid % kWave == 0) {
      rv[tid / kWave] = bv;
      ri[tid / kWave] = bi;
    }
    __syncthreads();
    bv = rv[0];
    bi = ri[0];
    for (int w = 1; w < kTokThreads / kWave; ++w)
      if (better(rv[w], ri[w], bv, bi)) {
        bv = rv[w];
        bi = ri[w];
      }
    next = bi < V ? bi : 0;  // every element was -inf: index 0, as torch.argmax
  }
  if (x_next != nullptr) {
    // the next step's input rows, as decode_embed_kernel forms them for the
    // token just chosen at position p + 1 (a NaN row for an id outside its
    // table), so that the next decode step needs no embedding launch
    const int64_t pn = p + 1;
    const bool ok = next >= 0 && next < emb_rows && pn >= 0 && pn < max_pos;
    const float4* e = (const float4*)emb + (ok ? next : 0) * d4;
    const float4* q = (const float4*)pos_emb + (ok ? pn : 0) * d4;
    float4* o = (float4*)x_next + b * d4;
    for (int j = tid; j < d4; j += kTokThreads) {
      const float4 a = e[j], c = q[j];
      o[j] = ok ? make_float4(a.x + c.x, a.y + c.y, a.z + c.z, a.w + c.w) : make_float4(NAN, NAN, NAN, NAN);
    }
  }
  if (tid == 0) {
    token[b] = next;
    const int64_t g = p + 1 - P;
    if (g >= 0 && g < out_cap) out[b * out_stride + g] = next;
    __threadfence();  // this workgroup's writes (and its read of *position, above) come first
    last = atomicAdd(done, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (last && tid == 0) {
    *position = p + 1;
    *done = 0u;  // ready for the next step
    __threadfence();
  }
}

// The decode step's input rows (model.py:29-127, the embedding and position
// embedding of one token per stream): out[b] = emb[token[b]] + pos_emb[*position],
// one fp32 add per element as the two indexings and the add compute it.  A
// workgroup of 64 threads per stream, one 16-byte vector per thread and pass.
// An id outside its table writes a NaN row.
__global__ __launch_bounds__(64) void decode_embed_kernel(const float* __restrict__ emb,
                                                          const float* __restrict__ pos_emb,
                                                          const int64_t* __restrict__ token,
                                                          const int64_t* __restrict__ position, int64_t vocab,
                                                          int64_t max_pos, int d4, float* __restrict__ out) {
  const int64_t b = blockIdx.x;
  const int64_t t = token[b], p = *position;
  const bool ok = t >= 0 && t < vocab && p >= 0 && p < max_pos;
  const float4* e = (const float4*)emb + (ok ? t : 0) * d4;
  const float4* q = (const float4*)pos_emb + (ok ? p : 0) * d4;
  float4* o = (float4*)out + b * d4;
  for (int j = threadIdx.x; j < d4; j += 64) {
    const float4 a = e[j], c = q[j];
    o[j] = ok ? make_float4(a.x + c.x, a.y + c.y, a.z + c.z, a.w + c.w) : make_float4(NAN, NAN, NAN, NAN);
  }
}

}  // namespace
}  // namespace mpl

using namespace mpl;

extern "C" int mpl_decode_next_token(const float* logits, int64_t rows, int64_t vocab, const int64_t* prompt,
                                     int64_t prompt_stride, const int64_t* prompt_len, int64_t* position,
                                     int64_t* token, int64_t* out, int64_t out_stride, int64_t out_cap,
                                     uint32_t* done, void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && vocab > 0 && prompt_stride >= 0 && out_cap >= 0 && out_stride >= 0, MPL_EINVAL,
              "mpl_decode_next_token: bad sizes rows=%lld vocab=%lld", (long long)rows, (long long)vocab);
  MPL_REQUIRE(rows < ((int64_t)1 << 31) && vocab < ((int64_t)1 << 31), MPL_EINVAL,
              "mpl_decode_next_token: rows=%lld or vocab=%lld too large", (long long)rows, (long long)vocab);
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(logits && prompt && prompt_len && position && token && done && (out || out_cap == 0), MPL_EINVAL,
              "mpl_decode_next_token: null buffer");
  next_token_kernel<<<(unsigned)rows, kTokThreads, 0, (hipStream_t)stream>>>(
      logits, vocab, prompt, prompt_stride, prompt_len, position, token, out, out_stride, out_cap, done, nullptr, 0,
      nullptr, 0, 0, nullptr);
  return check_launch("mpl_decode_next_token");
}

extern "C" int mpl_decode_next_token_embed(const float* logits, int64_t rows, int64_t vocab, const int64_t* prompt,
                                           int64_t prompt_stride, const int64_t* prompt_len, int64_t* position,
                                           int64_t* token, int64_t* out, int64_t out_stride, int64_t out_cap,
                                           uint32_t* done, const float* emb, int64_t emb_rows,
                                           const float* pos_emb, int64_t max_pos, int d, float* x_next,
                                           void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && vocab > 0 && prompt_stride >= 0 && out_cap >= 0 && out_stride >= 0 && emb_rows > 0 &&
                  max_pos > 0 && d > 0 && d % 4 == 0,
              MPL_EINVAL, "mpl_decode_next_token_embed: bad sizes rows=%lld vocab=%lld d=%d", (long long)rows,
              (long long)vocab, d);
  MPL_REQUIRE(rows < ((int64_t)1 << 31) && vocab < ((int64_t)1 << 31), MPL_EINVAL,
              "mpl_decode_next_token_embed: rows=%lld or vocab=%lld too large", (long long)rows, (long long)vocab);
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(logits && prompt && prompt_len && position && token && done && (out || out_cap == 0) && emb &&
                  pos_emb && x_next,
              MPL_EINVAL, "mpl_decode_next_token_embed: null buffer");
  MPL_REQUIRE(((uintptr_t)emb & 15) == 0 && ((uintptr_t)pos_emb & 15) == 0 && ((uintptr_t)x_next & 15) == 0,
              MPL_EINVAL, "mpl_decode_next_token_embed: emb, pos_emb and x_next must be 16-byte aligned");
  next_token_kernel<<<(unsigned)rows, kTokThreads, 0, (hipStream_t)stream>>>(
      logits, vocab, prompt, prompt_stride, prompt_len, position, token, out, out_stride, out_cap, done, emb,
      emb_rows, pos_emb, max_pos, d / 4, x_next);
  return check_launch("mpl_decode_next_token_embed");
}

extern "C" int mpl_decode_embed(const float* emb, int64_t vocab, const float* pos_emb, int64_t max_pos, int d,
                                const int64_t* token, const int64_t* position, int64_t rows, float* out,
                                void* stream) {
  clear_error();
  MPL_REQUIRE(rows >= 0 && vocab > 0 && max_pos > 0 && d > 0 && d % 4 == 0, MPL_EINVAL,
              "mpl_decode_embed: bad sizes rows=%lld vocab=%lld max_pos=%lld d=%d", (long long)rows,
              (long long)vocab, (long long)max_pos, d);
  MPL_REQUIRE(rows < ((int64_t)1 << 31), MPL_EINVAL, "mpl_decode_embed: rows=%lld too large", (long long)rows);
  if (rows == 0) return MPL_OK;
  MPL_REQUIRE(emb && pos_emb && token && position && out, MPL_EINVAL, "mpl_decode_embed: null buffer");
  MPL_REQUIRE(((uintptr_t)emb & 15) == 0 && ((uintptr_t)pos_emb & 15) == 0 && ((uintptr_t)out & 15) == 0,
              MPL_EINVAL, "mpl_decode_embed: emb, pos_emb and out must be 16-byte aligned");
  decode_embed_kernel<<<(unsigned)rows, 64, 0, (hipStream_t)stream>>>(emb, pos_emb, token, position, vocab, max_pos,
                                                                      d / 4, out);
  return check_launch("mpl_decode_embed");
}
