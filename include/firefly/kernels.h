// kernels.h - the paged KV-cache operators with the reference's call signatures.
//
// Drop-in for the KV-cache part of include/firefly/kernels.h (reference, :8-9 and :70-84):
//   set_default_stream / get_default_stream   thread-local stream every launch below uses
//   attention(...)                            paged decode when kv_cache_block_table != nullptr
//   apply_rope(...)                           rotary embedding of q and k (reference :68)
// plus the append the reference keeps private to its model (src/model/qwen_model.cu:21-47, launched at
// :138-143), exported here, a fused rope + append, and quantized-cache overloads.  Each forwards to the C ABI
// in ffkv.h.
//
// The reference's other operators (the model math, off this path) keep their declarations below unchanged, so
// that src/model/qwen_model.cu and src/engine.cc compile against this header; their definitions stay in the
// caller's own kernel files (src/kernels/{embedding,norm,activation,add,linear,sampling}.cu), which this
// library does not provide.  The caller drops the stream setter/getter its src/kernels/embedding.cu:41-45 defines
// (cudaStream_t): this library's set_default_stream / get_default_stream (hipStream_t) replace them.
//
// Like the reference, the functions return void and report failures on std::cerr
// (src/kernels/attention.cu:487-491); last_error() additionally returns the message of the calling thread's
// last failure ("" if none).  Everything is asynchronous on the default stream and may be captured in a hipGraph.
#pragma once

#include <hip/hip_runtime_api.h>

#include <string>

#include "firefly/tensor.h"

namespace firefly::kernels
{

FIREFLY_API void        set_default_stream(hipStream_t stream);
FIREFLY_API hipStream_t get_default_stream();
FIREFLY_API std::string last_error();

// The decode operators keep one split-K workspace per (thread, device, stream), held for the life of the thread
// (a graph captured on the stream has its address).  release_workspace(stream) synchronizes `stream` and frees
// the calling thread's workspace for it on the current device; call it when a stream is retired and no graph
// captured on it will be replayed again (the next call on that stream allocates a new one).  No counterpart in the
// reference, whose temporaries are stream-ordered allocations.
FIREFLY_API void release_workspace(hipStream_t stream);

// Bytes one pool block (16 tokens of one layer, K and V, scales included) takes for a cache dtype (F32, F16, BF16,
// I8, FP8_E4M3; 0 otherwise): the divisor of the engine's pool sizing (src/engine.cc:90-96), which assumes 2-byte
// elements.  fp8 caches add 2 * num_kv_heads * 4 bytes of per-head scales per layer.  ffkv_kv_block_bytes.
FIREFLY_API size_t kv_block_bytes(DType cache_dtype, int num_kv_heads, int head_dim);

/**
 * @brief Scaled dot-product attention (reference include/firefly/kernels.h:83-84).
 *
 * Paged decode when kv_cache_block_table != nullptr and q is [B, 1, Hq, D]: k / v the page pools
 * [num_blocks, 16, kv_head_num, D]; output [B, 1, Hq*D] (or any tensor of B*Hq*D elements) in q's dtype;
 * kv_cache_block_table int32 [B, max_context_blocks] on the device; context_lens int32 [B] on the device, tokens
 * cached before this step (context_lens[b] + 1 tokens are attended); seq_len is not used, as in the reference's
 * decode branch.
 *
 * Prefill otherwise (seq_len must equal q.shape()[1]; output [B, S, Hq*D]):
 *   - kv_cache_block_table == nullptr: the reference's contiguous causal prefill (src/kernels/attention.cu:460-474),
 *     k / v the chunk's [B, S, kv_head_num, D] tensors;
 *   - kv_cache_block_table != nullptr and S > 1: chunked prefill over the pages, query t of row b at position
 *     context_lens[b] + t attending keys 0 .. context_lens[b] + t (the chunk must already be appended), which
 *     reuses a cached prefix instead of recomputing it.
 */
FIREFLY_API void attention(Tensor& q, Tensor& k, Tensor& v, Tensor& output, void* kv_cache_block_table,
                           int kv_head_num, int seq_len, int max_context_blocks, const int* context_lens);

// Paged decode over an int8 (k_scale/v_scale fp32 [num_blocks, 16, Hkv]) or fp8 e4m3 (fp32 [Hkv]) cache.
FIREFLY_API void attention(Tensor& q, Tensor& k_cache, Tensor& v_cache, const Tensor& k_scale, const Tensor& v_scale,
                           Tensor& output, void* kv_cache_block_table, int kv_head_num, int seq_len,
                           int max_context_blocks, const int* context_lens);

/**
 * @brief Paged decode of a batch whose block tables share their first shared_blocks entries (radix-tree prefix
 * sharing): the shared pages are attended once for all rows (ffkv_paged_decode_shared_prefix).  Same tensors and
 * results as the decode branch of attention(); no counterpart in the reference, whose decode reads shared pages
 * once per row.  shared_blocks = 0 is the plain decode.
 */
FIREFLY_API void attention_shared_prefix(Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& output,
                                         void* kv_cache_block_table, int kv_head_num, int max_context_blocks,
                                         const int* context_lens, int shared_blocks);

/**
 * @brief The decode step's append_kv_cache(k, v, ...) followed by the decode branch of attention(q, ...), as one
 * call (ffkv_append_paged_decode): k / v [B, 1, kv_head_num, head_dim] are the step's new tokens, written to the
 * pages at context_lens[b] exactly as append_kv_cache writes them, and q [B, 1, Hq, head_dim] attends
 * context_lens[b] + 1 keys.  One kernel launch when k / v have the cache's 16-bit dtype, the two calls otherwise.
 * The reference runs the pair as two launches (src/model/qwen_model.cu:138-146); 16-bit caches only here (the
 * quantized caches take the scale-taking append_kv_cache and attention overloads).
 */
FIREFLY_API void append_kv_cache_attention(const Tensor& k, const Tensor& v, Tensor& q, Tensor& k_cache,
                                           Tensor& v_cache, Tensor& output, void* kv_cache_block_table,
                                           int kv_head_num, int max_context_blocks, const int* context_lens);

/**
 * @brief Write new K/V tokens into their pages (the reference's append_kv_cache kernel).
 *
 * k, v [B, S, Hkv, D] (F32/F16/BF16); k_cache, v_cache [num_blocks, 16, Hkv, D]; token t of row b goes to
 * position context_lens[b] + t (context_lens == nullptr means 0) of the row's block table
 * (block_table[b*max_blocks + pos/16], slot pos%16).  A narrower cache type rounds to nearest even.
 */
FIREFLY_API void append_kv_cache(const Tensor& k, const Tensor& v, Tensor& k_cache, Tensor& v_cache,
                                 const int* block_table, const int* context_lens, int max_blocks);

// Quantizing append: int8 cache (k_scale/v_scale written, fp32 [num_blocks, 16, Hkv]: absmax/127 per token and
// head) or fp8 e4m3 cache (k_scale/v_scale read, fp32 [Hkv] per head).
FIREFLY_API void append_kv_cache(const Tensor& k, const Tensor& v, Tensor& k_cache, Tensor& v_cache, Tensor& k_scale,
                                 Tensor& v_scale, const int* block_table, const int* context_lens, int max_blocks);

/**
 * @brief Rotary position embedding of q and k in place (reference include/firefly/kernels.h:68,
 * src/kernels/rope.cu:22-137).
 *
 * q [B, S, Hq, D] and k [B, S, Hkv, D] of one dtype (F32/F16/BF16); head_dim must equal D and seq_len S.  Token t
 * of row b is at position context_lens[b] + t (context_lens == nullptr: t); rotate-half pairs (i, i + D/2) turn by
 * position * theta^(-2i/D).  An empty q (no data) rotates k only.
 */
FIREFLY_API void apply_rope(Tensor& q, Tensor& k, int head_dim, int seq_len, float theta, const int* context_lens);

/**
 * @brief apply_rope(q, k, ...) then append_kv_cache(k, v, ...) in one kernel: the pair the reference's model runs
 * back to back (src/model/qwen_model.cu:136-143).  Pages are bit-identical to the two separate calls.
 */
FIREFLY_API void rope_append_kv_cache(Tensor& q, Tensor& k, const Tensor& v, Tensor& k_cache, Tensor& v_cache,
                                      const int* block_table, const int* context_lens, int max_blocks, float theta);

// Quantizing variant (k_scale/v_scale as for the quantizing append_kv_cache).
FIREFLY_API void rope_append_kv_cache(Tensor& q, Tensor& k, const Tensor& v, Tensor& k_cache, Tensor& v_cache,
                                      Tensor& k_scale, Tensor& v_scale, const int* block_table,
                                      const int* context_lens, int max_blocks, float theta);

// ---- the reference's off-path operators: declared as in its include/firefly/kernels.h, defined by the caller --

// Embedding lookup (reference include/firefly/kernels.h:18).
void embedding_lookup(const Tensor& input_ids, const Tensor& embedding_table, Tensor& output);

// RMS normalization (reference include/firefly/kernels.h:28).
void rms_norm(const Tensor& input, const Tensor& weight, Tensor& output, double epsilon);

// SwiGLU: silu(gate) * up (reference include/firefly/kernels.h:39).
void swiglu(const Tensor& gate, const Tensor& up, Tensor& output);

// x += y (reference include/firefly/kernels.h:47).
void add_inplace(Tensor& x, const Tensor& y);

// output = input * weight (reference include/firefly/kernels.h:56).
void matmul(const Tensor& input, const Tensor& weight, Tensor& output);

// Greedy sampling (reference include/firefly/kernels.h:92).
void argmax(const Tensor& logits, Tensor& output_token);

}  // namespace firefly::kernels
