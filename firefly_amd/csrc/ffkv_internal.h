// ffkv_internal.h - argument blocks and launchers shared by the C ABI layer and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ffkv
{

constexpr int kBlockSize = 16;  // tokens per KV page, fixed by the reference (include/firefly/scheduler.h:71)

struct AppendArgs
{
    const void*    k_src;
    const void*    v_src;
    void*          k_cache;
    void*          v_cache;
    float*         k_scale;
    float*         v_scale;
    const int32_t* block_table;
    const int32_t* context_lens;
    int            src_dtype;
    int            cache_dtype;
    int            batch;
    int            seq_len;
    int            num_kv_heads;
    int            head_dim;
    int            max_blocks;
    int            num_blocks;
};

struct RopeArgs
{
    void*          q;  // [B, S, Hq, D] rotated in place, or null (num_heads = 0)
    void*          k;  // [B, S, Hkv, D] rotated in place
    const void*    v;  // [B, S, Hkv, D], appended with k (when k_cache is set)
    void*          k_cache;  // null: rotate only
    void*          v_cache;
    float*         k_scale;
    float*         v_scale;
    const int32_t* block_table;
    const int32_t* context_lens;
    int            src_dtype;
    int            cache_dtype;
    int            batch;
    int            seq_len;
    int            num_heads;
    int            num_kv_heads;
    int            head_dim;
    int            max_blocks;
    int            num_blocks;
    float          theta;
};

struct PrefillArgs
{
    const void*    q;    // [B, S, Hq, D]
    void*          out;  // [B, S, Hq * D]
    const void*    k_cache;  // paged: [N, 16, Hkv, D]; contiguous: [B, S, Hkv, D]
    const void*    v_cache;
    const float*   k_scale;
    const float*   v_scale;
    const int32_t* block_table;   // paged only
    const int32_t* context_lens;  // paged only: tokens cached before the chunk
    int            qo_dtype;
    int            cache_dtype;
    int            batch;
    int            seq_len;
    int            num_heads;
    int            num_kv_heads;
    int            group;
    int            head_dim;
    int            max_blocks;
    int            num_blocks;
    int            cap_tokens;  // paged: keys per row are clamped to this
    bool           paged;
    float          scale_log2;
    // Shared-prefix partials (launch_prefix_partials) only: decode queries q [batch, 1, num_heads, head_dim] over
    // pages 0 .. pfx_blocks - 1 of block-table row 0, in pfx_chunks chunks of pfx_chunk_pages pages; the partial
    // of (row b, head h, chunk k) goes to decode-workspace slot pfx_slot0 + k * batch + b.
    int            pfx_blocks;
    int            pfx_chunks;
    int            pfx_chunk_pages;
    int            pfx_slot0;
    float*         ws_ml;
    float*         ws_acc;
};

struct DecodeArgs
{
    const void*    q;
    void*          out;
    const void*    k_cache;
    const void*    v_cache;
    const float*   k_scale;
    const float*   v_scale;
    const int32_t* block_table;
    const int32_t* context_lens;
    // Partial results.  Generic kernel: [batch, num_heads, max_chunks] entries.  MFMA kernel: slot = work item +
    // row, [items + batch, num_heads] entries.
    float*         ws_ml;   // [.., 2]: running max (log2 domain) and denominator
    float*         ws_acc;  // [.., head_dim]: unnormalised output
    int32_t*       ws_meta;  // MFMA kernel: [batch, 2] first and last work item covering each row
    int            qo_dtype;
    int            cache_dtype;
    int            batch;
    int            num_heads;
    int            num_kv_heads;
    int            group;  // num_heads / num_kv_heads
    int            head_dim;
    int            max_blocks;
    int            num_blocks;
    int            cap_tokens;  // attended tokens per row are clamped to this
    int            items;       // MFMA kernel: work items of the launch (decode_mfma_launch_items)
    int            chunk;       // tokens per split-K chunk (multiple of 16)
    int            max_chunks;  // ceil(cap_tokens / chunk)
    float          scale_log2;  // softmax scale * log2(e)
    // Shared-prefix mode (pfx_chunks > 0, MFMA kernel only): the first skip_blocks pages of every row are left to
    // launch_prefix_partials, whose pfx_chunks partials per row sit at slots pfx_slot0 + k * batch + b; the decode
    // kernel attends the remaining pages and writes partials only, and the merge folds both for every row.
    int            skip_blocks;
    int            pfx_chunks;
    int            pfx_slot0;
    // Fused shared-prefix launch (launch_decode_pfx): work items 0 .. pfx_items - 1 compute prefix partials first,
    // and their share of the rows' own pages is pfx_share / 1024 of another item's.  0 elsewhere.
    int            pfx_items;
    int            pfx_share;
    // Fused append (16-bit caches, k/v in the cache dtype): [batch, 1, num_kv_heads, head_dim]; the item holding a
    // row's last page takes the new token from here and writes it to its page slot (the first wave copies the
    // tokens of rows cut short by cap_tokens).
    const void*    k_new;
    const void*    v_new;
};

hipError_t launch_append(const AppendArgs& a, hipStream_t stream);
hipError_t launch_rope_append(const RopeArgs& a, hipStream_t stream);      // rotate q/k, then append when k_cache set
hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream);  // matrix-core prefill (16- and 8-bit caches)
hipError_t launch_prefix_partials(const PrefillArgs& a, hipStream_t stream);  // shared-prefix decode partials
hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream);       // generic kernel (any cache dtype)
hipError_t launch_decode_mfma(const DecodeArgs& a, hipStream_t stream);  // matrix-core kernel (16-bit/8-bit caches)
// Copies the first `width` ints of `rows` rows of `pitch` ints from src (pinned host memory mapped into the device's
// address space: its device pointer) to dst (device memory) with a kernel on `stream`.
hipError_t launch_staging_copy(int32_t* dst, const int32_t* src, int pitch, int width, int rows, hipStream_t stream);

// Upper bound on the MFMA kernel's work items (sizes its partial-result slots).
constexpr int kMfmaMaxItems = 2048;
// Work items for one MFMA decode launch: as many workgroups as the device keeps resident at once (CUs times
// occupancy of `kernel` at `threads` threads), divided over `grid_y` head groups, capped at kMfmaMaxItems.
int decode_mfma_items(const void* kernel, int threads, int grid_y);
// decode_mfma_items for the kernel instance launch_decode_mfma selects for `a` (its dtypes, head_dim and heads).
int decode_mfma_launch_items(const DecodeArgs& a);
bool decode_use_mfma(int cache_dtype, int group, int head_dim);

// Fused shared-prefix decode (paged_decode_pfx.hip): the prefix partials and the decode of the rows' own pages in
// one grid, then the merge.  decode_pfx_plan sizes it for `a` (dtypes, batch, heads, head_dim set) over
// `shared_pages` shared pages in at most `max_chunks` chunks, or returns false when the fused kernel does not take
// these dtypes / head_dim / heads (then the prefix kernel and the decode launch one after the other).
struct DecodePfxPlan
{
    int items;        // decode work items (grid x)
    int gy;           // head groups (grid y)
    int chunks;       // prefix chunks
    int chunk_pages;  // pages per prefix chunk
    int pfx_items;    // items that compute a prefix task first
    int pfx_share;    // their page share, per 1024 of another item's
};
constexpr int kPfxDefaultShare = 512;
bool       decode_pfx_plan(const DecodeArgs& a, int shared_pages, int max_chunks, DecodePfxPlan& plan);
hipError_t launch_decode_pfx(const DecodeArgs& a, const PrefillArgs& p, int gy, hipStream_t stream);
size_t decode_mfma_workspace_bytes(int batch, int num_heads, int head_dim);  // upper bound (kMfmaMaxItems items)

// Split-K geometry shared by the workspace query and the launcher.
int    decode_cap_tokens(int max_blocks, int max_context_len);
int    decode_min_chunk(int cap_tokens);
int    decode_chunk(int batch, int num_kv_heads, int cap_tokens);
size_t decode_workspace_bytes(int batch, int num_heads, int head_dim, int cap_tokens);

}  // namespace ffkv
