/*
 * ffkv.h - C ABI of the MI355X (gfx950) paged KV-cache path.
 *
 * This is the drop-in boundary for Firefly's paged KV-cache hot path: appending new K/V tokens into
 * block-table-addressed pages (optionally quantizing to int8 or OCP fp8 e4m3, optionally fused with the rotary
 * embedding of q and k) and PagedAttention decode (GQA, split-K, online softmax).  Plain pointers and sizes
 * only; no C++ or HIP types appear here, so ctypes / cgo / JNI / N-API callers can bind it directly.  `stream` is a hipStream_t passed as void*
 * (NULL = the legacy default stream).
 *
 * Layout contract (identical to the reference):
 *   K/V pages       [num_blocks, block_size=16, num_kv_heads, head_dim], element (p, o, h, d) at
 *                   ((p*16 + o)*num_kv_heads + h)*head_dim + d        (src/model/qwen_model.cu:41-42,
 *                                                                       src/kernels/attention.cu:347-348)
 *   block_table     int32 [batch, max_blocks], row stride max_blocks  (src/kernels/attention.cu:334)
 *   context_lens    int32 [batch], tokens already cached BEFORE this step's append
 *                   (src/model/qwen_model.cu:32-33, src/kernels/attention.cu:320)
 *   append source   [batch, seq_len, num_kv_heads, head_dim]          (src/model/qwen_model.cu:39)
 *   q               [batch, 1, num_heads, head_dim]; out [batch, 1, num_heads*head_dim]
 *   GQA head map    kv_head = q_head / (num_heads / num_kv_heads)     (src/kernels/attention.cu:304)
 *
 * Quantized caches (no counterpart in the reference, which is fp16-only):
 *   FFKV_DTYPE_I8       symmetric int8, scale per (page, slot, kv_head): fp32 [num_blocks, 16, num_kv_heads],
 *                       scale = absmax/127 (IEEE fp32 divide), q = clamp(rint_half_even(x/scale), -127, 127),
 *                       absmax == 0 gives scale 0 and q 0.  Scales are WRITTEN by ffkv_append.
 *   FFKV_DTYPE_FP8_E4M3 OCP e4m3 (bias 7, max 448, NaN = S.1111.111), scale per kv_head: fp32 [num_kv_heads],
 *                       q = e4m3_round_half_even_satfinite(x/scale).  Scales are READ by ffkv_append.
 *
 * Invalid addressing is defined instead of undefined (the reference writes/reads block -1 for padded rows,
 * src/engine.cc:298-300 with src/model/qwen_model.cu:37,41-45): a block-table entry < 0 or >= num_blocks,
 * a logical block index >= max_blocks, or a negative position is skipped by append and masked out by decode;
 * a decode row with no valid token produces zeros.
 *
 * All entry points are asynchronous on `stream`, never synchronize the host, and are safe to capture in a
 * hipGraph as long as a workspace is passed to ffkv_paged_decode.  Return 0 on success or a negative
 * FFKV_ERR_* code; ffkv_last_error() gives a message for the calling thread.
 */
#ifndef FFKV_H_
#define FFKV_H_

#include <stddef.h>
#include <stdint.h>

#ifndef FFKV_API
#define FFKV_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define FFKV_BLOCK_SIZE 16

/* dtype codes: equal to the firefly::DType enumerators F32, F16, BF16, I8 (include/firefly/types.h:16-26 in
 * the reference, whose enum continues I32, I64, U8, UNKNOWN = 7), plus FP8_E4M3 = 8, which the reference lacks. */
#define FFKV_DTYPE_F32 0
#define FFKV_DTYPE_F16 1
#define FFKV_DTYPE_BF16 2
#define FFKV_DTYPE_I8 3
#define FFKV_DTYPE_FP8_E4M3 8

#define FFKV_OK 0
#define FFKV_ERR_INVALID_ARGUMENT -1
#define FFKV_ERR_UNSUPPORTED -2
#define FFKV_ERR_WORKSPACE -3
#define FFKV_ERR_HIP -4

/*
 * Scatter new K/V tokens into their pages.  Replaces the reference's unexported append kernel launch
 * `append_kv_cache<<<(seq_len, Hkv, B), 128, 0, stream>>>(k, v, k_cache, v_cache, block_table, context_lens,
 * max_blocks, Hkv, D)` (src/model/qwen_model.cu:21-47, launched at :138-143).
 *
 * Token t of row b goes to position pos = context_lens[b] + t (context_lens == NULL means 0), i.e. page
 * block_table[b*max_blocks + pos/16], slot pos%16.  src_dtype is F32, F16 or BF16; cache_dtype is F32, F16,
 * BF16 (copy, rounding to nearest even when narrowing), I8 or FP8_E4M3 (quantize, see above).
 * k_scale / v_scale: I8 -> written, [num_blocks, 16, num_kv_heads]; FP8 -> read, [num_kv_heads]; else unused.
 * head_dim is a multiple of 8 up to 128 (the reference's append takes any head_dim up to its 128-thread block),
 * or 256; block_size must be 16.  Source and cache pointers must be 16-byte aligned.
 */
FFKV_API int ffkv_append(const void* k_src, const void* v_src, int src_dtype, void* k_cache, void* v_cache, int cache_dtype,
                float* k_scale, float* v_scale, const int32_t* block_table, const int32_t* context_lens, int batch,
                int seq_len, int num_kv_heads, int head_dim, int block_size, int max_blocks, int num_blocks,
                void* stream);

/*
 * Bytes one pool block (16 tokens of one layer, K and V) takes in a cache of cache_dtype, its scales included:
 * what an engine divides its memory budget by to size the pools.  Replaces the 16-bit element size in the
 * reference's `max_num_blocks = 0.9 * free / (num_layers * 16 * Hkv * D * 2 * 2)` (src/engine.cc:90-96, pools
 * allocated at :104-113):
 *   F32        16 * Hkv * D * 4 * 2
 *   F16, BF16  16 * Hkv * D * 2 * 2
 *   I8         16 * Hkv * (D + 4) * 2   codes and the per-token-per-head fp32 scales [num_blocks, 16, Hkv]
 *   FP8_E4M3   16 * Hkv * D * 2         codes; the per-head scales (2 * Hkv * 4 bytes per layer) do not grow
 *                                       with the pool
 * Returns 0 for another dtype or a non-positive size.  No counterpart in the reference (fp16 pools only).
 */
FFKV_API size_t ffkv_kv_block_bytes(int cache_dtype, int num_kv_heads, int head_dim);

/*
 * Bytes of scratch ffkv_paged_decode needs for split-K partial results at these sizes.  max_context_len is
 * an upper bound on context_lens[b] + 1 (<= 0 means max_blocks * 16).  No counterpart in the reference, whose
 * decode kernel has no split-K (src/kernels/attention.cu:475-485).
 */
FFKV_API size_t ffkv_decode_workspace_bytes(int batch, int num_heads, int head_dim, int max_blocks, int max_context_len);


/*
 * PagedAttention decode: out[b, h, :] = softmax(scale * q[b,h] . K_j) V_j over the context_lens[b] + 1 cached
 * tokens of row b (the +1 is the token appended this step).  Replaces `firefly::kernels::attention(q, k_cache,
 * v_cache, out, block_table, kv_head_num, seq_len, max_context_blocks, context_lens)` on its decode branch
 * (include/firefly/kernels.h:83-84, src/kernels/attention.cu:452-493 -> paged_attention_kernel :291-447).
 *
 * qo_dtype (q and out) is F32, F16 or BF16; cache_dtype as for ffkv_append.  scale <= 0 selects
 * 1/sqrt(head_dim) (src/kernels/attention.cu:458).  num_heads must be a multiple of num_kv_heads (any group
 * size for 16- and 8-bit caches at head_dim 64, 80, 96, 112, 128 and 256, at most 16 otherwise)
 * and at most 65535; head_dim a multiple of 8 up to 128 (as the reference's decode,
 * src/kernels/attention.cu:307-316), or 256: 64, 80, 96, 112, 128 and 256 run the matrix-core kernels, the others a
 * vector kernel; q, out, cache and workspace pointers 16-byte aligned.  Rows are
 * split over the context and the pieces merged; the partials live in `workspace` (ffkv_decode_workspace_bytes;
 * any initial contents), or, when workspace is NULL, in stream-ordered memory the library allocates and frees on
 * `stream`.  Calls sharing one workspace must not overlap in time (use one workspace per stream).  Rows whose
 * context_lens[b] + 1 exceeds max_context_len are truncated to it.
 */
FFKV_API int ffkv_paged_decode(const void* q, void* out, int qo_dtype, const void* k_cache, const void* v_cache,
                      int cache_dtype, const float* k_scale, const float* v_scale, const int32_t* block_table,
                      const int32_t* context_lens, int batch, int num_heads, int num_kv_heads, int head_dim,
                      int block_size, int max_blocks, int num_blocks, int max_context_len, float scale,
                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * ffkv_paged_decode without any device allocation: the split-K partials live in a static scratch array that the
 * library holds on every GPU it runs on (FFKV_NOALLOC_SCRATCH_BYTES each, until the process ends), so the call
 * never allocates or frees device memory, whatever `workspace` contract the caller could keep.  No counterpart in
 * the reference; it is for callers that cannot allocate: code under hipGraph capture, tight serving loops, hosts
 * that forbid allocation after start-up.  Arguments and results are those of ffkv_paged_decode (same kernels, same
 * split, bit-identical outputs).  Sizes whose partials exceed the scratch (roughly (work items + batch) *
 * num_heads * (head_dim + 2) * 4 bytes with the matrix-core kernel, batch * num_heads * chunks * (head_dim + 2) *
 * 4 with fp32 caches) return FFKV_ERR_WORKSPACE.  All calls on one GPU share its scratch: calls that overlap in
 * time on one GPU (two streams, two threads) race and must be serialized by the caller.
 */
#define FFKV_NOALLOC_SCRATCH_BYTES (32u << 20)

FFKV_API int ffkv_paged_decode_noalloc(const void* q, void* out, int qo_dtype, const void* k_cache,
                                       const void* v_cache, int cache_dtype, const float* k_scale,
                                       const float* v_scale, const int32_t* block_table, const int32_t* context_lens,
                                       int batch, int num_heads, int num_kv_heads, int head_dim, int block_size,
                                       int max_blocks, int num_blocks, int max_context_len, float scale,
                                       void* stream);

/*
 * ffkv_append of one token per row (seq_len 1) followed by ffkv_paged_decode, as one call: the decode step of
 * the reference's model (src/model/qwen_model.cu:138-146, append launch then kernels::attention).  k_new / v_new
 * [batch, 1, num_kv_heads, head_dim] in src_dtype; the other arguments as for the two functions.  When the
 * step's k/v already have the cache's 16-bit type it is a single launch: the decode work item that holds a
 * row's last page reads the new token from k_new / v_new instead of the page, attends it, and writes it to its
 * page slot (rows cut short by max_context_len get the token copied to its slot without attending it).
 * Otherwise it runs the two functions in turn.  Either way the pages are
 * bit-identical to ffkv_append's and the output is ffkv_paged_decode's on them.  No counterpart in the
 * reference (two launches there).
 */
FFKV_API int ffkv_append_paged_decode(const void* k_new, const void* v_new, int src_dtype, const void* q, void* out,
                                      int qo_dtype, void* k_cache, void* v_cache, int cache_dtype, float* k_scale,
                                      float* v_scale, const int32_t* block_table, const int32_t* context_lens,
                                      int batch, int num_heads, int num_kv_heads, int head_dim, int block_size,
                                      int max_blocks, int num_blocks, int max_context_len, float scale,
                                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * ffkv_paged_decode for a batch whose rows share a prefix of pages (the radix tree's shared blocks): entries
 * 0 .. shared_blocks - 1 of every row's block table are the same physical pages, read from row 0's table.  The
 * prefix is attended once for all rows as a matrix product (every row's queries of a kv head against each
 * prefix page, split into chunks of pages), the rest of each row by the decode kernel, and the split-K merge
 * folds both: each shared page is read once per call instead of once per row.  Results equal ffkv_paged_decode
 * on the same inputs up to floating-point summation order (same tolerance).  Rows shorter than the prefix
 * attend only their own tokens.  The split applies to F16/BF16/I8/FP8 caches; fp32 caches run
 * ffkv_paged_decode unchanged.  No counterpart in the reference, whose decode reads shared blocks once per row
 * (src/kernels/attention.cu:332-335).  Workspace: ffkv_decode_shared_prefix_workspace_bytes, or NULL as for
 * ffkv_paged_decode.
 */
FFKV_API size_t ffkv_decode_shared_prefix_workspace_bytes(int batch, int num_heads, int num_kv_heads, int head_dim,
                                                          int max_blocks, int max_context_len, int shared_blocks);

FFKV_API int ffkv_paged_decode_shared_prefix(const void* q, void* out, int qo_dtype, const void* k_cache,
                                             const void* v_cache, int cache_dtype, const float* k_scale,
                                             const float* v_scale, const int32_t* block_table,
                                             const int32_t* context_lens, int batch, int num_heads, int num_kv_heads,
                                             int head_dim, int block_size, int max_blocks, int num_blocks,
                                             int max_context_len, float scale, int shared_blocks, void* workspace,
                                             size_t workspace_bytes, void* stream);

/*
 * Causal prefill attention over the paged cache (chunked prefill with prefix reuse).  Replaces the prefill branch
 * of `firefly::kernels::attention` (kv_cache_block_table == nullptr: flash_attn_wmma_kernel,
 * src/kernels/attention.cu:22-286, dispatched at :460-474) and extends it to cached prefixes, which the
 * reference's model skips (src/model/qwen_model.cu:147-151 routes every multi-token batch-1 step to the
 * contiguous kernel).
 *
 * q [batch, seq_len, num_heads, head_dim], out [batch, seq_len, num_heads*head_dim], both qo_dtype.  With a
 * block table, query token t of row b sits at position context_lens[b] + t and attends the row's keys
 * 0 .. context_lens[b] + t read from the pages (context_lens = tokens cached BEFORE this chunk, whose K/V must
 * already be appended, e.g. by ffkv_append with the same context_lens); keys on invalid pages or at or beyond
 * min(context_lens[b] + seq_len, max_context_len or max_blocks*16) are skipped, and a query with no key gives
 * zeros.  With block_table == NULL, k_cache / v_cache are the chunk's contiguous [batch, seq_len, num_kv_heads,
 * head_dim] tensors and positions start at 0: the reference's causal prefill.  seq_len = 1 is decode attention.
 * cache_dtype F16, BF16, I8 or FP8_E4M3 (scales as for ffkv_paged_decode); any GQA group; scale <= 0 selects
 * 1/sqrt(head_dim).  No workspace; pointers 16-byte aligned.  fp8 per-head K scales may be any finite value (0
 * weighs the keys uniformly, a negative one negates the scores, as in decode).  int8 caches: the attention
 * weights (below 2^8) meet their V scales in f16, so a per-token V scale of 256 or more can overflow; a workgroup
 * whose results overflow reruns with its weights scaled by 2^-12, which takes V scales up to 2^20 (|V| up to about
 * 1.3e8).  bf16 caches: V enters the products in f16 (a workgroup that meets |V| >= 65520 reruns in bf16), so V values
 * below 2^-14 carry an absolute error of at most 2^-25.  16-bit caches: an infinite V value also makes NaN, in
 * its dim, the outputs of the queries whose causal limit masks its key (it meets them with weight 0 in the tile
 * products), as in the reference's prefill, whose P.V tile product (src/kernels/attention.cu:232-243) takes every
 * key of its 16-key tile, the causally masked ones with p = 0 (:173-174).
 */
FFKV_API int ffkv_paged_prefill(const void* q, void* out, int qo_dtype, const void* k_cache, const void* v_cache,
                                int cache_dtype, const float* k_scale, const float* v_scale, const int32_t* block_table,
                                const int32_t* context_lens, int batch, int seq_len, int num_heads, int num_kv_heads,
                                int head_dim, int block_size, int max_blocks, int num_blocks, int max_context_len,
                                float scale, void* stream);

/*
 * Rotary position embedding of q and k in place.  Replaces `firefly::kernels::apply_rope(q, k, head_dim, seq_len,
 * theta, context_lens)` (include/firefly/kernels.h:68, src/kernels/rope.cu:22-137, called at
 * src/model/qwen_model.cu:136).  q [batch, seq_len, num_heads, head_dim] and k [batch, seq_len, num_kv_heads,
 * head_dim] share `dtype` (F32, F16 or BF16); q may be NULL (then num_heads is ignored).  Token t of row b is
 * at position context_lens[b] + t (t when context_lens is NULL).  Rotate-half form: pair i (dims i, i + D/2) is
 * rotated by pos * inv_freq_i with inv_freq_i = theta^(-2i/head_dim):
 *     x_i' = x_i cos - x_{i+D/2} sin,   x_{i+D/2}' = x_{i+D/2} cos + x_i sin.
 * inv_freq, cos and sin are evaluated in double precision and rounded once to fp32, the angle is one fp32
 * product of float(pos) and inv_freq, the rotation uses separately rounded fp32 products and sums, and the
 * result is rounded to nearest even in `dtype`.  q and k must be 16-byte aligned.
 */
FFKV_API int ffkv_rope(void* q, void* k, int dtype, const int32_t* context_lens, int batch, int seq_len, int num_heads,
                       int num_kv_heads, int head_dim, float rope_theta, void* stream);

/*
 * ffkv_rope followed by ffkv_append of the rotated k (as rounded in src_dtype) and v, in one pass: the
 * reference's `kernels::apply_rope` + append launch pair (src/model/qwen_model.cu:136-143) fused, saving a
 * launch and a read of k.  Arguments as for ffkv_rope and ffkv_append; q may be NULL.  k is rotated in place
 * (as apply_rope leaves it) and v is only read.  The page contents are bit-identical to ffkv_rope followed by
 * ffkv_append.
 */
FFKV_API int ffkv_rope_append(void* q, void* k, const void* v, int src_dtype, void* k_cache, void* v_cache,
                              int cache_dtype, float* k_scale, float* v_scale, const int32_t* block_table,
                              const int32_t* context_lens, int batch, int seq_len, int num_heads, int num_kv_heads,
                              int head_dim, int block_size, int max_blocks, int num_blocks, float rope_theta,
                              void* stream);

/* Message describing the last error returned on the calling thread ("" if none). */
FFKV_API const char* ffkv_last_error(void);

/* Library version string. */
FFKV_API const char* ffkv_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FFKV_H_ */
