/*
 * mpl.h -- C ABI of the MI355X (gfx950) memory-layer lookup library
 * (libmpl.so, built from the HIP sources in model_amd/csrc).
 *
 * The reference (KumarDev7/model) has no FFI: its operator is the Flax module
 * `MemoryPool` (memory_pool_model/memory.py:64-227) plus the trainer's sparse
 * row update (memory_pool_model/train.py:146-172, 395-426).  Each entry point
 * below replaces one stage of that module, cited per function.  A JAX
 * integration registers thin XLA FFI handlers over these functions; the
 * Python host mirror in model_amd/ calls them through ctypes.
 *
 * Conventions (all entry points):
 *   - plain device pointers and sizes; `stream` is a hipStream_t (NULL = the
 *     null stream) passed as void*;
 *   - no entry point allocates device memory or synchronises the stream;
 *     scratch comes from a caller-owned workspace sized by the matching
 *     *_workspace_bytes() query;
 *   - return 0 on success, otherwise an MPL_E* code, with a message for the
 *     calling thread in mpl_last_error();
 *   - scalars that change from step to step in training (the clamped
 *     temperature, the routing-noise coefficient) are device fp32 scalars
 *     (`const float*`), so a training step needs no host read and can be
 *     captured in a HIP graph;
 *   - tensors are dense row-major in the shapes given; M = number of query
 *     tokens, H = heads, n = sub-keys per codebook, half = d_key / 2,
 *     k = top_k, N = n*n slots, d = d_value.
 */
#ifndef MPL_H
#define MPL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MPL_F32 = 0, MPL_F16 = 1 };
enum { MPL_OK = 0, MPL_EINVAL = 1, MPL_EHIP = 2, MPL_EWORKSPACE = 3, MPL_EUNSUPPORTED = 4 };

/* query_mode of mpl_score_select */
enum { MPL_Q_NORMALIZED = 0, MPL_Q_RAW = 1, MPL_Q_RAW_SCALED = 2 };

/* activation and weight_layout of mpl_rows_linear */
enum { MPL_ACT_NONE = 0, MPL_ACT_GELU_TANH = 1, MPL_ACT_SILU = 2 };
enum { MPL_W_IN_OUT = 0, MPL_W_OUT_IN = 1 };

/* Library version (major*10000 + minor*100 + patch). */
int mpl_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* mpl_last_error(void);

/*
 * memory.py:30-31 and 136-139: y = x * rsqrt(sum(x*x) + eps) over rows of
 * length `dim`.  x, y: [rows, dim] fp32 (may alias).  If y16 != NULL it also
 * receives y rounded to fp16 (the query operand of fp16 scoring).  If
 * row_len != NULL it receives sqrt(sum(x*x) + eps) / sqrt(dim) per row: the
 * q_len of memory.py:137 (used when query_scale is on).
 */
int mpl_l2_normalize(const float* x, int64_t rows, int dim, float eps, float* y,
                     void* y16, float* row_len, void* stream);

/*
 * memory.py:139: normalise sub_keys [H,2,n,half] (fp32) and pack them into
 * the MFMA operand layout consumed by mpl_score_select, in one pass.
 * keys_hat [H,2,n,half] fp32 (optional, NULL = not written) receives the
 * normalised keys (the backward needs them).  score_dtype selects the
 * scoring precision: MPL_F16 (fp16 MFMA, fp32 accumulate) or MPL_F32 (fp32
 * MFMA).  `packed` must hold mpl_packed_keys_bytes() bytes.
 */
size_t mpl_packed_keys_bytes(int H, int n, int half, int score_dtype);
int mpl_pack_keys(const float* sub_keys, int H, int n, int half, int score_dtype,
                  float* keys_hat, void* packed, void* stream);

/*
 * memory.py:136-178: cosine scores of the queries [M,H,2,half] against the
 * packed keys, times `temperature` (a device fp32 scalar, already clamped,
 * memory.py:143-146) and,
 * with query_scale, times q_len (memory.py:151-152).  `queries` is either
 *   query_mode MPL_Q_NORMALIZED: unit rows in score_dtype (fp16 for MPL_F16,
 *     fp32 for MPL_F32, e.g. from mpl_l2_normalize); q_len [M,H,2] is an
 *     input (NULL = no query_scale);
 *   MPL_Q_RAW / MPL_Q_RAW_SCALED (fp16 scoring only): the raw fp32 queries,
 *     l2-normalised inside the kernel (memory.py:30-31, 136); with
 *     MPL_Q_RAW_SCALED the scores are also scaled by
 *     q_len = sqrt(sum q^2 + 1e-6) / sqrt(half), written to q_len if not NULL.
 * Optional routing noise select = scores + noise_coef *
 * gumbel with gumbel [M,H,2,n] fp32 (memory.py:155-159, NULL = no noise)
 * and noise_coef a device fp32 scalar (routing_noise * noise_scale; read
 * only with gumbel);
 * exact stage-1 top-k per codebook (ties: lowest sub-key index), exact
 * stage-2 top-k over the k*k candidates (ties: lowest flat index
 * rank_a*k + rank_b, memory.py:171), softmax of the clean slot scores.
 * Outputs (descending select order):
 *   sub_idx    [M,H,2,k] int32   stage-1 sub-key ids   (memory.py:162)
 *   sub_scores [M,H,2,k] fp32    clean sub scores      (memory.py:163)
 *   flat_idx   [M,H,k]   int32   rank_a*k + rank_b     (memory.py:171)
 *   slots      [M,H,k]   int32   idx_a*n + idx_b       (memory.py:175)
 *   weights    [M,H,k]   fp32    softmax               (memory.py:178)
 * Requires 1 <= k <= min(n, 32), 1 <= half <= 128, n*n < 2^31.
 */
size_t mpl_score_select_workspace_bytes(int64_t M, int H, int n, int half, int k);
int mpl_score_select(const void* queries, int query_mode, float* q_len, const void* packed_keys,
                     int64_t M, int H, int n, int half, int k, int score_dtype,
                     const float* temperature, const float* gumbel, const float* noise_coef,
                     void* workspace, size_t workspace_bytes,
                     int32_t* sub_idx, float* sub_scores, int32_t* flat_idx,
                     int32_t* slots, float* weights, void* stream);

/*
 * memory.py:132-193 (MemoryPool.__call__'s forward read, model.py:112-113):
 * mpl_score_select followed by the value read of mpl_gather_wsum, in one
 * call.  Same arguments, workspace (mpl_score_select_workspace_bytes) and
 * outputs as mpl_score_select, plus values [n*n, d] in values_dtype (MPL_F16
 * or MPL_F32), shuffle_reads (memory.py:179) and out [M, d] fp32, which equal
 * mpl_gather_wsum(values, values_dtype, n*n, d, slots, weights, M, H*k,
 * shuffle_reads, out) bit for bit.  With H = 4 and k = 16 the pair stage and
 * the value read run in one kernel (one wave per token) when the key range is
 * scored in at most 8 splits or reduced to 8 lists.
 */
int mpl_lookup(const void* queries, int query_mode, float* q_len, const void* packed_keys,
               int64_t M, int H, int n, int half, int k, int score_dtype,
               const float* temperature, const float* gumbel, const float* noise_coef,
               void* workspace, size_t workspace_bytes,
               int32_t* sub_idx, float* sub_scores, int32_t* flat_idx,
               int32_t* slots, float* weights,
               const void* values, int values_dtype, int d, int shuffle_reads,
               float* out, void* stream);

/*
 * Row files of the host tier's file mode (host_pool.py:90-108, 117-165: the
 * reference's .npy memmaps, read and written by numpy on host threads).  A
 * row file is `rows` rows of `row_bytes` bytes starting at byte data_offset
 * of the file at `path` (the data of an .npy array).  mpl_rowfile_read copies
 * rows ids[0..count) into dst (packed, in id order); mpl_rowfile_write
 * writes src's packed rows to those ids; both split the list over up to
 * `threads` host threads, copying through a shared mapping of the file
 * (runs of consecutive ids as one copy; mpl_rowfile_sync makes written rows
 * durable).  Ids outside [0, rows) fail with MPL_EINVAL
 * before any transfer.  dst/src are host memory (pinned memory lets the GPU
 * use it directly).  Host code only: no device work, no stream.
 */
int mpl_rowfile_open(const char* path, int64_t data_offset, int64_t row_bytes, int64_t rows, int writable,
                     void** handle);
int mpl_rowfile_read(void* handle, const int64_t* ids, int64_t count, void* dst, int threads);
/* The reads of host_pool.py:117-127 (HostPool.gather of a file-backed pool)
 * without the page cache: as mpl_rowfile_read, through a descriptor of the
 * file opened with O_DIRECT; each thread reads the 4 KiB-aligned spans around
 * its rows (neighbouring spans merged into reads of up to 1 MiB) and copies
 * the rows out, so rows come from the drive and nothing stays cached.
 * MPL_EUNSUPPORTED where the file system refuses O_DIRECT (tmpfs);
 * mpl_rowfile_direct_supported tells beforehand (1 or 0). */
int mpl_rowfile_read_direct(void* handle, const int64_t* ids, int64_t count, void* dst, int threads);
int mpl_rowfile_direct_supported(void* handle);
int mpl_rowfile_write(void* handle, const int64_t* ids, int64_t count, const void* src, int threads);
int mpl_rowfile_sync(void* handle);
/* host_pool.py:190-204: writes the file's dirty rows back, then asks the OS to
 * drop its pages from the page cache (advisory), so the next reads come from
 * the drive. */
int mpl_rowfile_evict(void* handle);
int mpl_rowfile_close(void* handle);

/*
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc).
 * mpl_lookup with the same arguments and outputs, minus the workspace: the
 * selection's scratch is a fixed array of mpl_lookup_static_scratch_bytes()
 * (32 MiB) on each GPU, held until the process ends; a lookup needing more
 * (mpl_score_select_workspace_bytes above it, e.g. beyond about 65,000 tokens
 * at n = 512) fails with MPL_EWORKSPACE.  Calls on one GPU share that array:
 * calls that overlap in time on one GPU (other streams, other threads) race.
 * Nothing is allocated; the current device must be the stream's device
 * (checked: MPL_EINVAL otherwise).
 */
size_t mpl_lookup_static_scratch_bytes(void);
int mpl_lookup_static(const void* queries, int query_mode, float* q_len, const void* packed_keys,
                      int64_t M, int H, int n, int half, int k, int score_dtype,
                      const float* temperature, const float* gumbel, const float* noise_coef,
                      int32_t* sub_idx, float* sub_scores, int32_t* flat_idx,
                      int32_t* slots, float* weights,
                      const void* values, int values_dtype, int d, int shuffle_reads,
                      float* out, void* stream);

/*
 * memory.py:161-163 and 207 (_top_k of the select scores, or of the clean
 * scores for the balance loss's f): stage 1 of mpl_score_select alone, same
 * arguments and semantics, writing only sub_idx [M,H,2,k] and sub_scores
 * [M,H,2,k] (clean scores, descending select order).  With several key
 * splits the split lists are reduced to one; the workspace query includes
 * that scratch.
 */
size_t mpl_score_topk_workspace_bytes(int64_t M, int H, int n, int half, int k);
int mpl_score_topk(const void* queries, int query_mode, float* q_len, const void* packed_keys,
                   int64_t M, int H, int n, int half, int k, int score_dtype,
                   const float* temperature, const float* gumbel, const float* noise_coef,
                   void* workspace, size_t workspace_bytes,
                   int32_t* sub_idx, float* sub_scores, void* stream);

/*
 * memory.py:156 (jax.random.gumbel(rng, scores.shape)): fills out [rows, n]
 * fp32 (rows = M*H*2 for the gumbel input of mpl_score_select) with
 * Gumbel(0,1) samples g = -log(-log(u)), u on JAX's grid {k * 2^-23} of
 * [FLT_MIN, 1), from a counter-based hash of (seed, row, column): each
 * element depends only on those three, so the fill is one write pass and
 * reproducible from the seed.  The stream differs from JAX's PRNG (the
 * distribution and support are the same).
 */
int mpl_gumbel_noise(uint64_t seed, int64_t rows, int n, float* out, void* stream);

/*
 * Synthetic tables of the pool's shapes, defined by a hash so that the CPU
 * can regenerate any rows of a table larger than host memory (the values
 * init of memory.py:104-109 is jax.random.normal; this stands in for it in
 * benchmarks).  Fills out [rows, cols] (dtype MPL_F16 or MPL_F32) with the
 * elements of table rows row0 .. row0 + rows - 1:
 *   index = row * cols + col, h = splitmix64(splitmix64(seed) ^ index),
 *   u1 = ((h >> 40) + 1) / 2^24, u2 = (h & 0xFFFFFF) / 2^24,
 *   value = (dtype)(float)(sqrt(-2 ln u1) cos(2 pi u2) * scale), in fp64.
 * splitmix64: the SplitMix64 finalizer (Steele, Lea & Flood 2014).
 */
int mpl_hash_normal_fill(void* out, int dtype, int64_t rows, int cols, uint64_t seed, float scale, int64_t row0,
                         void* stream);

/*
 * memory.py:179-193: out[m,:] = sum_r weights[m,r] * values[read(slots[m,r]),:]
 * over the R = H*k rows of each token, fp32 accumulation; values [N,d] in
 * values_dtype (MPL_F16 or MPL_F32); read(s) = s, or (s + N/2 + 1) % N when
 * shuffle_reads != 0 (memory.py:179).  out: [M,d] fp32.
 */
int mpl_gather_wsum(const void* values, int values_dtype, int64_t N, int d,
                    const int32_t* slots, const float* weights, int64_t M, int R,
                    int shuffle_reads, float* out, void* stream);

/*
 * host_pool.py:206-220 (fetch: jnp.unique(flat, size=P, return_inverse=True)
 * on the device before the host read): uniq [P] int32 receives the distinct
 * slots ascending, then pool_size for u >= U; inverse [P] int32 the position
 * of slots[p] in uniq (uniq[inverse[p]] == slots[p]); num_unique [1] (device)
 * U.  Slots are expected in [0, pool_size); other values are tolerated
 * (never out of bounds) but not sorted meaningfully.  Workspace of
 * mpl_unique_slots_workspace_bytes() bytes.
 */
size_t mpl_unique_slots_workspace_bytes(int64_t P, int64_t pool_size);
int mpl_unique_slots(const int32_t* slots, int64_t P, int64_t pool_size, void* workspace,
                     size_t workspace_bytes, int32_t* uniq, int32_t* inverse, int32_t* num_unique,
                     void* stream);

/*
 * host_pool.py:117-127 (HostPool.gather: rows of the table for the given
 * ids) as one device kernel: out[i, :] = table[clamp(idx[i]), :] for
 * i < min(count, *count_dev) (count_dev, device memory, may be NULL), rows
 * of d elements of dtype (MPL_F16 / MPL_F32) copied unchanged; ids are
 * clamped to [0, N).  The table may be device memory or pinned host memory
 * mapped for the device (its device address from mpl_host_device_pointer):
 * the kernel then reads the rows across the host link.
 */
int mpl_gather_rows(const void* table, int dtype, int64_t N, int d, const int32_t* idx,
                    int64_t count, const int32_t* count_dev, void* out, void* stream);

/*
 * No counterpart in the reference (which reads host rows on host threads):
 * the device address of pinned host memory (hipHostGetDevicePointer), for
 * passing a pinned table to mpl_gather_rows, mpl_row_adagrad or
 * mpl_row_adam.  Fails, without launching anything, for memory that is not
 * pinned and mapped.
 */
int mpl_host_device_pointer(void* host_ptr, void** dev_ptr);

/*
 * train.py:146-172 (fetched_row_grads + _merge_rows): gradient rows of the
 * fetched pool rows.  Fetch p in [0, P) of token p / fetches_per_token reads
 * slot slots[p] with weight weights[p] (weights == NULL: 1).  With
 * cap = min(P, pool_size) it writes
 *   uniq       [cap]    int32  distinct slots ascending, then pool_size padding
 *   rows       [cap,d]  fp32   sum over the fetches of uniq[u] of
 *                              weights[p] * g[p / fetches_per_token, :]; 0 for padding
 *   row_sq     [cap]    fp32   squared L2 norm of each row (for the global clip)
 *   num_unique [1]      int32  number of distinct slots (device memory)
 * g: [P / fetches_per_token, d] fp32.  Several memory layers are merged by
 * stacking their tokens (slots/weights concatenated in the same order).
 * Passing the materialised contributions as g with fetches_per_token = 1 and
 * weights = NULL is _merge_rows itself.  Deterministic: a stable radix sort
 * by slot and fixed-order segment sums, no float atomics.  Needs d <= 1024,
 * P and pool_size < 2^31, slots in [0, pool_size).  zero_padding = 0 leaves
 * rows [num_unique, cap) unwritten (uniq and row_sq are still padded), for
 * callers that skip padding slots, such as mpl_row_adagrad / mpl_row_adam.
 */
size_t mpl_merge_rows_workspace_bytes(int64_t P, int d, int64_t pool_size);
int mpl_merge_rows(const int32_t* slots, const float* weights, int64_t P, int fetches_per_token,
                   const float* g, int d, int64_t pool_size, void* workspace, size_t workspace_bytes,
                   int32_t* uniq, float* rows, float* row_sq, int32_t* num_unique, int zero_padding,
                   void* stream);

/*
 * mpl_merge_rows that also writes slot_counts [pool_size] fp32, the number of
 * fetches of every slot (memory.py:215: zeros(pool_size).at[slots].add(1),
 * summed over the merged layers as model.py:136 sums the layers' counts),
 * from the segments of the same sort: no atomics.  It replaces the per-fetch
 * histogram of mpl_route_counts for a training step that merges the fetched
 * rows anyway.  No counterpart in the reference (which takes the counts from
 * the forward's aux).  Same workspace as mpl_merge_rows.
 */
int mpl_merge_rows_counts(const int32_t* slots, const float* weights, int64_t P, int fetches_per_token,
                          const float* g, int d, int64_t pool_size, void* workspace, size_t workspace_bytes,
                          int32_t* uniq, float* rows, float* row_sq, int32_t* num_unique, int zero_padding,
                          float* slot_counts, void* stream);

/*
 * train.py:395-397: gnorm = sqrt(rest_sq + sum(row_sq)) and
 * scale = min(1, grad_clip / (gnorm + 1e-6)); scale_gnorm[0] = scale,
 * scale_gnorm[1] = gnorm (device memory).  rest_sq (device, may be NULL = 0)
 * is the squared global norm of the dense gradients.  The sum is taken in a
 * fixed order in fp64 (two stages, workspace of
 * mpl_clip_scale_workspace_bytes()).
 */
size_t mpl_clip_scale_workspace_bytes(void);
int mpl_clip_scale(const float* row_sq, int64_t cap, const float* rest_sq, float grad_clip,
                   float* scale_gnorm, void* workspace, size_t workspace_bytes, void* stream);

/*
 * mpl_clip_scale with the dense gradients' squared norm taken in the same
 * pass (train.py:395-397: optax.global_norm over every gradient): the sum
 * of row_sq [cap] plus the squares of the count (< 8) dense buffers x[j]
 * of n[j] fp32 each, in fp64 in a fixed order, then scale_gnorm as
 * mpl_clip_scale writes it.  Workspace as mpl_clip_scale.  It replaces
 * mpl_sum_squares + mpl_clip_scale (two launches fewer).  No counterpart in
 * the reference's interface.
 */
int mpl_clip_scale_dense(const float* row_sq, int64_t cap, const float* const* x, const int64_t* n, int count,
                         float grad_clip, float* scale_gnorm, void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * train.py:395-397 (the dense part of optax.global_norm's square):
 * out[0] = (add ? add[0] : 0) + sum over the count <= 8 fp32 buffers
 * x[j] [n[j]] of x^2.  x and n are host arrays of device pointers and sizes.
 * fp64 accumulation in a fixed order (256 chunks of the joined buffers, then
 * one block): bitwise reproducible, no atomics and no memset, so it may be
 * captured in a HIP graph.  workspace: mpl_sum_squares_workspace_bytes().
 */
size_t mpl_sum_squares_workspace_bytes(void);
int mpl_sum_squares(const float* const* x, const int64_t* n, int count, const float* add, float* out,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * train.py:412-416 (row-wise Adagrad, in place): for each u < cap with
 * 0 <= uniq[u] < pool_size (padding is dropped), g = rows[u] * grad_scale,
 * acc' = acc[s] + mean(g^2), values[s] += -lr / (sqrt(acc') + 1e-8) * g,
 * acc[s] = acc'.  values [pool_size, d] in values_dtype; with master != NULL
 * (fp32 [pool_size, d]) the master takes the update and values receives its
 * cast (host_pool.py:152 semantics for fp16 tables otherwise).  grad_scale:
 * device scalar or NULL (= 1), e.g. scale_gnorm from mpl_clip_scale.
 */
int mpl_row_adagrad(void* values, int values_dtype, float* master, float* acc,
                    const int32_t* uniq, const float* rows, int64_t cap, int d,
                    int64_t pool_size, float lr, const float* grad_scale, void* stream);

/*
 * train.py:417-426 (lazy Adam on the fetched rows, in place): m, v
 * [pool_size, d] fp32; b1 = 0.9, b2 = 0.999, eps = 1e-8; bias corrections
 * with n = step + 1 (step = the 0-based TrainState.step).  values, master,
 * grad_scale and padding as for mpl_row_adagrad.
 */
int mpl_row_adam(void* values, int values_dtype, float* master, float* m, float* v,
                 const int32_t* uniq, const float* rows, int64_t cap, int d,
                 int64_t pool_size, float lr, int step, const float* grad_scale, void* stream);

/*
 * Backward of the lookup (XLA's derivative of memory.py:136-193, written
 * out).  Route part: dw[m,r] = <g_out[m], values[read(slots[m,r])]>
 * (memory.py:192), the softmax backward ds = w (dw - sum w dw) per head
 * (:178) and its scatter to the stage-1 ranks, d_sub[m,h,0,flat/k] and
 * d_sub[m,h,1,flat%k] (:167-175), in j order.  g_out [M,d] fp32; slots,
 * weights, flat_idx [M,H,k] and sub_scores [M,H,2,k] from mpl_score_select;
 * read() as in mpl_gather_wsum.  Writes d_sub [M,H,2,k], d_weights [M,H,k]
 * (dw, optional) and dlogt_part [M] = sum over the token of
 * d_sub * sub_scores (the token's share of d log_temperature: T is the
 * straight-through clamp of memory.py:143-146).  Needs H*k <= 128.
 */
int mpl_lookup_bwd_route(const float* g_out, const void* values, int values_dtype, int64_t N, int d,
                         const int32_t* slots, const float* weights, const int32_t* flat_idx,
                         const float* sub_scores, int64_t M, int H, int k, int shuffle_reads,
                         float* d_weights, float* d_sub, float* dlogt_part, void* stream);

/*
 * d_queries [M,H,2,half] (the raw queries' gradient): dq_hat = sum_i
 * d_sub_i * T * q_len * k_hat[hc, sub_idx_i] + dq_hat_extra (optional dense
 * part [M,H,2,half], e.g. the balance loss), then the backward of
 * x * rsqrt(sum x^2 + 1e-6) (memory.py:30-31) and, with q_len != NULL
 * (query_scale), of q_len = sqrt(sum q^2 + 1e-6) / sqrt(half) (memory.py:137)
 * with d q_len = sum_i d_sub_i * sub_scores_i / q_len + dlen_extra (optional
 * [M,H,2]).  q: raw queries [M,H,2,half] fp32; k_hat [H,2,n,half] fp32
 * (mpl_pack_keys).  half <= 128.
 */
int mpl_lookup_bwd_queries(const float* q, const float* q_len, const float* k_hat,
                           const int32_t* sub_idx, const float* d_sub, const float* sub_scores,
                           const float* dq_hat_extra, const float* dlen_extra, int64_t M, int H,
                           int n, int half, int k, const float* temperature, float* d_queries, void* stream);

/*
 * d_sub_keys [H,2,n,half] (the raw sub_keys' gradient): dk_hat[hc,key] =
 * sum over the (m, i) that selected key of d_sub * T * q_len * q_hat[m,hc]
 * (a deterministic sort-by-key segmented sum, mpl_merge_rows) +
 * dk_hat_extra (optional dense part), then the l2-normalisation backward
 * against the raw sub_keys [H,2,n,half].  q_hat [M,H,2,half] fp32.
 */
size_t mpl_lookup_bwd_keys_workspace_bytes(int64_t M, int H, int n, int half, int k);
int mpl_lookup_bwd_keys(const float* sub_keys, const float* q_hat, const float* q_len,
                        const int32_t* sub_idx, const float* d_sub, const float* dk_hat_extra,
                        int64_t M, int H, int n, int half, int k, const float* temperature,
                        void* workspace, size_t workspace_bytes, float* d_sub_keys, void* stream);

/*
 * memory.py:143-146: t[0] = exp(clip(log_t[0], log_min, log_max)) as a
 * device scalar (a NaN log_t gives NaN), the clamped temperature of the
 * lookup, in one launch and no host read.
 */
int mpl_temperature(const float* log_t, float log_min, float log_max, float* t, void* stream);

/*
 * Backward of mpl_l2_normalize's y = x * rsqrt(sum(x*x) + eps) over rows of
 * length dim: dx = (dy - y (y . dy)) / sqrt(sum(x*x) + eps), multiplied by
 * *scale (a device scalar) when scale != NULL.  x, dy, dx: [rows, dim] fp32.
 * The derivative of memory.py:30-31 (XLA autodiff in the reference).
 */
int mpl_l2_normalize_bwd(const float* x, const float* dy, int64_t rows, int dim, float eps,
                         const float* scale, float* dx, void* stream);

/*
 * key_diversity_loss (memory.py:230-240): with G[h,c] = K_hat K_hat^T the
 * cosine Gram matrix of each codebook, loss [1] = sum of the squared
 * off-diagonal entries / (H * 2 * n * (n - 1)), the Gram tiles on MFMA in
 * score_dtype: MPL_F16 (half % 8 == 0, half <= 128) or MPL_F32 (half <=
 * 128).  If d_k_hat [H,2,n,half] != NULL it receives
 * d loss / d k_hat = 4 / (H * 2 * n * (n - 1)) * (G - diag G) K_hat (the
 * raw sub-keys' gradient follows with mpl_l2_normalize_bwd).  k_hat and
 * packed_keys from mpl_pack_keys with the same score_dtype.
 */
size_t mpl_key_diversity_workspace_bytes(int H, int n, int half, int score_dtype);
int mpl_key_diversity(const float* k_hat, const void* packed_keys, int H, int n, int half, int score_dtype,
                      void* workspace, size_t workspace_bytes, float* loss, float* d_k_hat, void* stream);

/*
 * revive_dead_keys (memory.py:243-281), in place: in every codebook the
 * sub-keys with usage < threshold / n (sub_keys [H,2,n,half], subkey_usage
 * [H,2,n], both fp32) become l2-normalise(queries[pick, h, c] + noise *
 * normal) with usage 1/n, and each codebook's usage is divided by its new
 * sum.  queries [M,H,2,half] (unit-norm query halves); the random draws of
 * memory.py:269-274 are inputs: pick [H,2,n] int32 in [0, M), normal
 * [H,2,n,half] fp32 standard normal.  dead [H,2,n] (uint8, optional)
 * receives the mask.  The trainer's reset of the optimizer moments of
 * revived keys (train.py:497-509) stays with the caller.
 */
int mpl_revive_keys(float* sub_keys, float* subkey_usage, const float* queries, int64_t M, const int32_t* pick,
                    const float* normal, int H, int n, int half, float threshold, float noise, uint8_t* dead,
                    void* stream);

/* *out = sum(x[0, n)) (+ *add if add != NULL), fixed order, fp64 accumulation. */
int mpl_sum(const float* x, int64_t n, const float* add, float* out, void* stream);

/*
 * memory.py:199-204, 206-208, 215: routing counts from the selected ids.
 *   subkey_counts [H,2,n] (or NULL): per codebook, how often each sub-key is
 *     an index of a final slot (slots [M,H,k] int32: slot = a*n + b counts
 *     a in codebook 0 and b in codebook 1 of its head);
 *   clean_counts [H,2,n] (or NULL): occurrences of each sub-key in
 *     clean_sub_idx [M,H,2,k] (the clean stage-1 ids; f = counts / (M k));
 *   slot_counts [n*n] (or NULL): occurrences of each slot in `slots`.
 * Outputs are overwritten.  Counts are fp32 whole numbers, exact (and so
 * independent of the order of the additions) while below 2^24.  Ids outside
 * their range are not counted.
 */
int mpl_route_counts(const int32_t* slots, const int32_t* clean_sub_idx, int64_t M, int H, int n, int k,
                     float* subkey_counts, float* clean_counts, float* slot_counts, void* stream);

/*
 * memory.py:209-213: the load-balance loss
 *   balance = n * mean_{h,c} sum_n f[h,c,n] * mean_m softmax_n(z[m,h,c,:])
 * with z = cos(q, k_n) * T * (q_len if scaled), f = clean_counts / (M k), the
 * cosine on MFMA tiles of score_dtype (MPL_F16: half % 8 == 0, half <= 128;
 * MPL_F32: half <= 128) and each softmax taken over all n sub-keys in one
 * online pass.  `scaled` = balance_temperature_grad && query_scale (the
 * balance logits are then the query-scaled scores).  queries: raw fp32
 * [M,H,2,half] (normalised inside).  packed_keys: from mpl_pack_keys with
 * score_dtype.  `state` (mpl_balance_state_bytes) receives per (token,
 * codebook) the softmax statistics that mpl_lookup_bwd_dense needs; loss [1]
 * (NaN when M = 0: f and the token mean are then 0/0, as in the reference).
 */
size_t mpl_balance_state_bytes(int64_t M, int H);
int mpl_balance_fwd(const float* queries, int scaled, const void* packed_keys, const float* clean_counts,
                    int64_t M, int H, int n, int half, int k, int score_dtype, const float* temperature, void* state,
                    float* loss, void* stream);

/*
 * The dense-over-n part of the lookup backward on MFMA tiles of score_dtype
 * (as mpl_balance_fwd) that recompute the scores:
 *   dk_hat [H,2,n,half], written: d/d(normalised sub-keys) of
 *     - the routed term (sub_idx, d_sub [M,H,2,k] non-NULL): the selected
 *       scores' gradient d_sub * T (* q_len with query_scale) against the
 *       normalised queries (memory.py:149-163 under XLA autodiff);
 *     - the balance term (g_balance non-NULL, a device scalar): the
 *       derivative of memory.py:209-213 with f held constant;
 *   dq_hat [M,H,2,half], written when g_balance != NULL: the balance term's
 *     d/d(normalised queries) (the routed d q_hat stays with
 *     mpl_lookup_bwd_queries, whose dq_hat_extra this is);
 *   with balance_temperature_grad and g_balance: dlen [M,H,2]
 *     (query_scale only) and dlogt [1], the balance's d q_len and d log_t
 *     shares.
 * q_hat from mpl_l2_normalize; k_hat and packed_keys from mpl_pack_keys
 * (score_dtype); clean_counts and state from mpl_route_counts / mpl_balance_fwd
 * of the same inputs; q_len [M,H,2] with query_scale.  The raw sub-keys'
 * gradient follows with mpl_l2_normalize_bwd.  Nothing of size [M, n] is
 * formed; no atomics.
 */
/*
 * One decode step of the backbone's causal self-attention with its
 * key/value cache (model.py:29-91 in decode mode, called once per token by
 * generate.py:31-34; Flax's MultiHeadDotProductAttention with decode=True).
 * qkv [batch, 3, heads, head_dim] fp32 is the fused query/key/value
 * projection of the new token of each stream (biases added), position a
 * device int64 scalar shared by every stream.  Writes the new key to
 * k_cache_t [batch, heads, head_dim, max_len] and the new value to
 * v_cache [batch, heads, max_len, head_dim] at that position, then
 * out [batch, heads, head_dim] = softmax_t((scale * q) . k_t) v_t over
 * t <= position.  head_dim is 16, 32, 64, 128 or 256; max_len <= 8192.  A position
 * outside [0, max_len) writes nothing to the caches and NaN to out.
 */
int mpl_decode_attention(const float* qkv, int64_t batch, int heads, int head_dim, int max_len,
                         const int64_t* position, float* k_cache_t, float* v_cache, float* out, float scale,
                         void* stream);

/*
 * The greedy generator's token step (generate.py:44-61) on the GPU, so that
 * a decode step and its token choice replay as one HIP graph.  For each of
 * `rows` streams, with p = *position and P = *prompt_len (device int64
 * scalars): the next token is prompt[b, p + 1] while p + 1 < P (prompt
 * [rows, prompt_stride] int64, P <= prompt_stride), else the first index of
 * the maximum of logits[b, 0..vocab) (fp32; NaN counts as the maximum, as
 * torch.argmax); it is written to token[b], and generated tokens to
 * out[b, p + 1 - P] (out [rows, out_stride] int64, indices >= out_cap
 * dropped).  Then *position becomes p + 1.  `done` is a device uint32 that
 * must be 0 before the first call; each call leaves it 0.  Calls on one
 * `done` must not overlap.
 */
int mpl_decode_next_token(const float* logits, int64_t rows, int64_t vocab, const int64_t* prompt,
                          int64_t prompt_stride, const int64_t* prompt_len, int64_t* position, int64_t* token,
                          int64_t* out, int64_t out_stride, int64_t out_cap, uint32_t* done, void* stream);

/*
 * mpl_decode_next_token that also writes the next decode step's input rows:
 * x_next[b] = emb[next token of b] + pos_emb[p + 1], with p the position it
 * read, the same bits as mpl_decode_embed at that token and position (a NaN
 * row for an id outside emb [emb_rows, d] or pos_emb [max_pos, d]; d % 4 ==
 * 0, the three 16-byte aligned).  A greedy generator whose step graph reads
 * x_next instead of embedding its tokens saves that launch per step.  No
 * counterpart in the reference's interface.
 */
int mpl_decode_next_token_embed(const float* logits, int64_t rows, int64_t vocab, const int64_t* prompt,
                                int64_t prompt_stride, const int64_t* prompt_len, int64_t* position, int64_t* token,
                                int64_t* out, int64_t out_stride, int64_t out_cap, uint32_t* done, const float* emb,
                                int64_t emb_rows, const float* pos_emb, int64_t max_pos, int d, float* x_next,
                                void* stream);

/*
 * The input rows of a decode step (model.py:29-127: the token embedding plus
 * the position embedding, for one token per stream): for each of `rows`
 * streams, out[b, :] = emb[token[b], :] + pos_emb[*position, :] (emb
 * [vocab, d] and pos_emb [max_pos, d] fp32, token int64 [rows], position a
 * device int64 scalar, out [rows, d] fp32).  d is a multiple of 4 and emb,
 * pos_emb and out are 16-byte aligned.  The same bits as the two indexings
 * and the add.  A token outside [0, vocab) or a position outside
 * [0, max_pos) writes a NaN row.
 */
int mpl_decode_embed(const float* emb, int64_t vocab, const float* pos_emb, int64_t max_pos, int d,
                     const int64_t* token, const int64_t* position, int64_t rows, float* out, void* stream);

/*
 * A dense layer of the backbone over a few rows (model.py:29-127: the
 * query/key/value, output, feed-forward, router, gate and mem_out products
 * and embed.attend), with its neighbours fused in:
 *   a = x [rows, K] fp32;  a = LayerNorm(a) * ln_scale + ln_bias if ln_scale
 *   (mean and biased variance over K, ln_eps inside the square root);
 *   a = a * x_mul if x_mul [rows, K];
 *   out [rows, N] = act(a . W + bias) + residual
 * W is [K, N] (MPL_W_IN_OUT, a Dense kernel) or [N, K] (MPL_W_OUT_IN, the
 * embedding table of embed.attend); bias [N], residual [rows, N] and x_mul
 * may be NULL; activation MPL_ACT_NONE, MPL_ACT_GELU_TANH
 * (0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))) or MPL_ACT_SILU.
 * K is a multiple of 4; x, x_mul, W, ln_scale and ln_bias are 16-byte
 * aligned; out may be the residual but not x or x_mul.  Deterministic.
 */
int mpl_rows_linear(const float* x, const float* x_mul, const float* ln_scale, const float* ln_bias, float ln_eps,
                    const float* weight, int weight_layout, const float* bias, int activation,
                    const float* residual, int64_t rows, int K, int N, float* out, void* stream);

/*
 * Two dense layers of the same (layer-normalised) rows as one product: the
 * memory layer's router and gate (model.py:110 and 118, both on
 * h = LayerNorm(x), model.py:98).  weight [K, N1 + N2] is the two
 * Dense kernels side by side (MPL_W_IN_OUT), bias [N1 + N2] (or NULL);
 *   out1 [rows, N1] = act1(a . weight[:, :N1] + bias[:N1])
 *   out2 [rows, N2] = act2(a . weight[:, N1:] + bias[N1:])
 * with a as in mpl_rows_linear (no x_mul, no residual).  Each output equals
 * mpl_rows_linear of its layer bit for bit.  No counterpart in the
 * reference's interface: it saves a decode step one launch per memory layer.
 */
int mpl_rows_linear_pair(const float* x, const float* ln_scale, const float* ln_bias, float ln_eps,
                         const float* weight, const float* bias, int activation1, int activation2, int64_t rows,
                         int K, int N1, int N2, float* out1, float* out2, void* stream);

/*
 * The output layer of a decode step (model.py:125-126): logits [rows, V] =
 * LayerNorm(x) . emb^T (ln_final, then embed.attend), x [rows, d], emb
 * [V, d] (x, ln_scale, ln_bias and emb 16-byte aligned), LayerNorm as in mpl_rows_linear (mean and
 * biased variance over d, ln_eps inside the square root), products on fp32
 * MFMA.  rows <= 64 and d a multiple of 4 up to 256 (MPL_EUNSUPPORTED
 * otherwise).  Deterministic.  No counterpart in the reference's interface:
 * it replaces a LayerNorm launch and a library GEMM in the decode step.
 */
int mpl_vocab_logits(const float* x, const float* ln_scale, const float* ln_bias, float ln_eps, const float* emb,
                     int64_t rows, int d, int64_t V, float* logits, void* stream);

size_t mpl_lookup_bwd_dense_workspace_bytes(int64_t M, int H, int n, int half, int score_dtype);
int mpl_lookup_bwd_dense(const float* q_hat, const float* q_len, const float* k_hat, const void* packed_keys,
                         const int32_t* sub_idx, const float* d_sub, const float* clean_counts, const void* state,
                         const float* g_balance, int balance_temperature_grad, int query_scale, int64_t M, int H,
                         int n, int half, int k, int score_dtype, const float* temperature, void* workspace,
                         size_t workspace_bytes, float* dq_hat, float* dk_hat, float* dlen, float* dlogt,
                         void* stream);

/*
 * The dense backward of a training step in one call (memory.py:136-164 and
 * 208-213; train.py's key diversity term, memory.py:230-240): what
 * mpl_lookup_bwd_dense, mpl_lookup_bwd_queries, mpl_key_diversity and the two
 * l2 normalisation backwards of the sub-keys compute, with fewer passes.
 *  - d_queries [M, 2H, half] fp32: the gradient with respect to the raw
 *    queries.  The routed d q_hat (d_sub * T at each query's k selected
 *    sub-keys) joins the balance term in the dense query pass, on the
 *    fp16 / fp32 MFMA operand at the sub-key pass's scale, and the pass ends
 *    with the l2 normalisation backward (eps as in mpl_lookup_bwd_queries).
 *  - d_sub_keys [2H, n, half] fp32: the gradient with respect to the raw
 *    sub_keys (fp32 [2H, n, half]) of the routed and balance terms, plus
 *    *g_diversity times that of key_diversity_loss when g_diversity (a device
 *    scalar) is given; the diversity loss then goes to diversity_loss [1].
 *    The diversity Gram pass reuses this call's key packs; its workspace is
 *    div_workspace (mpl_key_diversity_workspace_bytes).
 * queries are the raw queries (16-byte aligned when half % 4 == 0), q_hat
 * their normalisation, or NULL with fp16 scoring at half = 64 or 128: the
 * operand packs then normalise the raw queries themselves, to the same bits
 * as mpl_l2_normalize.  Only with the balance term, without query_scale or
 * balance_temperature_grad, k <= 16 and half <= 128 (MPL_EUNSUPPORTED
 * otherwise).  Workspace as mpl_lookup_bwd_dense.  phase = 0 runs it all;
 * phase = 1 only the query side (operand packs, scales, the query pass:
 * d_queries is complete when it returns to the stream) and phase = 2 the
 * sub-key side from what phase 1 left in the same workspace, so that a
 * caller can start work that needs d_queries (the projection's weight
 * gradient) on another stream between the two calls, which take the same
 * arguments.  No counterpart in the reference's interface (XLA fuses its
 * own backward): it saves the separate routed query pass, the fp32 q_hat
 * pass and the split sums.
 */
int mpl_lookup_bwd_dense_queries(const float* q_hat, const float* queries, const float* k_hat,
                                 const void* packed_keys, const int32_t* sub_idx, const float* d_sub,
                                 const float* clean_counts, const void* state, const float* g_balance, int64_t M,
                                 int H, int n, int half, int k, int score_dtype, const float* temperature,
                                 void* workspace, size_t workspace_bytes, float eps, float* d_queries,
                                 const float* sub_keys, const float* g_diversity, void* div_workspace,
                                 size_t div_workspace_bytes, float* diversity_loss, float* d_sub_keys, int phase,
                                 void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MPL_H */
