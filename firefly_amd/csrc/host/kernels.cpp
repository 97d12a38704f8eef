// kernels.cpp - firefly::kernels entry points over the C ABI (ffkv.h).
//
// Shapes and conventions follow the reference dispatcher (src/kernels/attention.cu:452-493): batch = q.shape[0],
// num_heads = q.shape[2], head_dim = q.shape[3], scale = 1/sqrt(head_dim), the block-table row stride is the
// max_context_blocks argument, and the launch goes to the thread's default stream.  The decode workspace (split
// partial results) is cached per (thread, device, stream) and grown outside of stream capture; while a stream is
// being captured a missing or too-small workspace makes the library allocate stream-ordered memory inside the graph
// instead.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <iostream>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "ffkv.h"
#include "firefly/kernels.h"

namespace firefly::kernels
{

namespace
{

thread_local hipStream_t t_stream = nullptr;
thread_local std::string t_error;

void report(int rc, const char* what)
{
    if (rc == FFKV_OK)
    {
        t_error.clear();
        return;
    }
    t_error = std::string(what) + ": " + ffkv_last_error();
    std::cerr << t_error << std::endl;
}

void fail(const std::string& msg)
{
    t_error = msg;
    std::cerr << msg << std::endl;
}

// Decode workspaces (split-K partials), one per (thread, device, stream): calls on different streams never share
// one, so a graph replayed on one stream does not race with eager calls on another.  A workspace that must grow is
// replaced by a larger one (at least twice the size) and the old buffer is retired, never freed: a graph captured
// while it was current has its address baked in and may still be replayed.  Retired buffers are therefore held
// until the process ends; the geometric growth keeps them smaller in total than the live one.  A thread that ends
// retires its live workspaces the same way.  release_workspace() frees a stream's workspace when the caller
// retires the stream (a host that makes a stream per request would otherwise hold one workspace per stream it
// ever used).  Nothing here synchronizes the device except release_workspace().
struct Workspace
{
    void*  ptr = nullptr;
    size_t bytes = 0;
};

std::mutex         g_retired_mu;
std::vector<void*> g_retired;  // never freed (see above)

struct WorkspaceCache
{
    std::map<std::pair<int, hipStream_t>, Workspace> by_stream;
    ~WorkspaceCache()  // thread exit: graphs captured by this thread may still hold these addresses
    {
        std::lock_guard<std::mutex> lock(g_retired_mu);
        for (const auto& kv : by_stream)
            if (kv.second.ptr != nullptr) g_retired.push_back(kv.second.ptr);
    }
};
thread_local WorkspaceCache t_ws;

// A workspace of at least `bytes` for the current device and the default stream, or nullptr while that stream is
// being captured and its workspace is too small (the library then allocates stream-ordered memory inside the
// graph instead; allocating here would be an unsafe call during capture).
void* workspace(size_t bytes, size_t& have)
{
    int dev = 0;
    (void)hipGetDevice(&dev);
    Workspace& ws = t_ws.by_stream[{dev, t_stream}];
    if (ws.ptr != nullptr && ws.bytes >= bytes)
    {
        have = ws.bytes;
        return ws.ptr;
    }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(t_stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
    {
        have = 0;
        return nullptr;
    }
    const size_t grow = std::max(bytes, 2 * ws.bytes);
    void*        p = nullptr;
    if (hipMalloc(&p, grow) != hipSuccess)
    {
        have = 0;
        return nullptr;
    }
    if (ws.ptr != nullptr)
    {
        std::lock_guard<std::mutex> lock(g_retired_mu);
        g_retired.push_back(ws.ptr);
    }
    ws = Workspace{p, grow};
    have = grow;
    return p;
}

bool is_gpu(const Tensor& t) { return t.device() == Device::GPU; }

}  // namespace

size_t kv_block_bytes(DType cache_dtype, int num_kv_heads, int head_dim)
{
    return ffkv_kv_block_bytes(static_cast<int>(cache_dtype), num_kv_heads, head_dim);
}

void release_workspace(hipStream_t stream)
{
    int dev = 0;
    (void)hipGetDevice(&dev);
    const auto it = t_ws.by_stream.find({dev, stream});
    if (it == t_ws.by_stream.end()) return;
    if (it->second.ptr != nullptr)
    {
        // the stream's queued work may still use it
        if (hipStreamSynchronize(stream) != hipSuccess || hipFree(it->second.ptr) != hipSuccess)
        {
            std::lock_guard<std::mutex> lock(g_retired_mu);  // keep it rather than free memory still in use
            g_retired.push_back(it->second.ptr);
            fail("release_workspace: could not synchronize the stream; the workspace is kept");
        }
    }
    t_ws.by_stream.erase(it);
}

namespace
{

int code(DType d) { return static_cast<int>(d); }

void decode(Tensor& q, Tensor& k, Tensor& v, const float* k_scale, const float* v_scale, Tensor& out,
            void* block_table, int kv_head_num, int max_context_blocks, const int* context_lens, int shared_blocks = 0)
{
    if (q.shape().size() != 4 || k.shape().size() != 4 || !is_gpu(q) || !is_gpu(k) || !is_gpu(v) || !is_gpu(out))
        return fail("PagedAttention: q must be [B, S, Hq, D] and all tensors on the GPU");
    const int B = static_cast<int>(q.shape()[0]);
    const int Hq = static_cast<int>(q.shape()[2]);
    const int D = static_cast<int>(q.shape()[3]);
    if (out.numel() < static_cast<int64_t>(B) * Hq * D || out.dtype() != q.dtype())
        return fail("PagedAttention: output must hold B*Hq*D elements of q's dtype");
    if (k.shape()[2] != kv_head_num || k.shape()[3] != D || v.shape() != k.shape() || v.dtype() != k.dtype())
        return fail("PagedAttention: k/v caches must both be [num_blocks, 16, kv_head_num, head_dim]");
    const size_t need = shared_blocks > 0 ? ffkv_decode_shared_prefix_workspace_bytes(B, Hq, kv_head_num, D,
                                                                                       max_context_blocks, 0,
                                                                                       shared_blocks)
                                          : ffkv_decode_workspace_bytes(B, Hq, D, max_context_blocks, 0);
    size_t       have = 0;
    void*        ws = workspace(need, have);
    const int rc = ffkv_paged_decode_shared_prefix(
        q.data(), out.data(), code(q.dtype()), k.data(), v.data(), code(k.dtype()), k_scale, v_scale,
        reinterpret_cast<const int32_t*>(block_table), context_lens, B, Hq, kv_head_num, D, FFKV_BLOCK_SIZE,
        max_context_blocks, static_cast<int>(k.shape()[0]), 0, 0.0f, shared_blocks, ws, have, t_stream);
    report(rc, "PagedAttention failed");
}

// Prefill: block_table == nullptr is the reference's contiguous causal branch (k, v [B, S, Hkv, D],
// src/kernels/attention.cu:460-474); otherwise chunked prefill over the paged cache with the chunk's queries at
// context_lens[b] + t.
void prefill(Tensor& q, Tensor& k, Tensor& v, const float* k_scale, const float* v_scale, Tensor& out,
             void* block_table, int kv_head_num, int seq_len, int max_context_blocks, const int* context_lens)
{
    if (q.shape().size() != 4 || k.shape().size() != 4 || !is_gpu(q) || !is_gpu(k) || !is_gpu(v) || !is_gpu(out))
        return fail("attention (prefill): q must be [B, S, Hq, D] and all tensors on the GPU");
    const int B = static_cast<int>(q.shape()[0]);
    const int S = static_cast<int>(q.shape()[1]);
    const int Hq = static_cast<int>(q.shape()[2]);
    const int D = static_cast<int>(q.shape()[3]);
    if (seq_len != S) return fail("attention (prefill): seq_len must equal q.shape()[1]");
    if (out.numel() < static_cast<int64_t>(B) * S * Hq * D || out.dtype() != q.dtype())
        return fail("attention (prefill): output must hold B*S*Hq*D elements of q's dtype");
    if (k.shape()[2] != kv_head_num || k.shape()[3] != D || v.shape() != k.shape() || v.dtype() != k.dtype())
        return fail("attention (prefill): k/v must be [.., .., kv_head_num, head_dim] and alike");
    if (block_table == nullptr && (k.shape()[0] != B || k.shape()[1] != S))
        return fail("attention (prefill): contiguous k/v must be [B, seq_len, kv_head_num, head_dim]");
    const int rc = ffkv_paged_prefill(q.data(), out.data(), code(q.dtype()), k.data(), v.data(), code(k.dtype()),
                                      k_scale, v_scale, reinterpret_cast<const int32_t*>(block_table), context_lens, B,
                                      S, Hq, kv_head_num, D, FFKV_BLOCK_SIZE, block_table ? max_context_blocks : 0,
                                      block_table ? static_cast<int>(k.shape()[0]) : 0, 0, 0.0f, t_stream);
    report(rc, "attention (prefill) failed");
}

void append(const Tensor& k, const Tensor& v, Tensor& kc, Tensor& vc, float* ks, float* vs, const int* block_table,
            const int* context_lens, int max_blocks)
{
    if (k.shape().size() != 4 || kc.shape().size() != 4 || v.shape() != k.shape() || vc.shape() != kc.shape() ||
        k.shape()[2] != kc.shape()[2] || k.shape()[3] != kc.shape()[3])
        return fail("append_kv_cache: k/v must be [B, S, Hkv, D] and the caches [num_blocks, 16, Hkv, D]");
    const int rc =
        ffkv_append(k.data(), v.data(), code(k.dtype()), kc.data(), vc.data(), code(kc.dtype()), ks, vs,
                    reinterpret_cast<const int32_t*>(block_table), reinterpret_cast<const int32_t*>(context_lens),
                    static_cast<int>(k.shape()[0]), static_cast<int>(k.shape()[1]), static_cast<int>(k.shape()[2]),
                    static_cast<int>(k.shape()[3]), static_cast<int>(kc.shape()[1]), max_blocks,
                    static_cast<int>(kc.shape()[0]), t_stream);
    report(rc, "append_kv_cache failed");
}

void rope_append(Tensor& q, Tensor& k, const Tensor* v, Tensor* kc, Tensor* vc, float* ks, float* vs,
                 const int* block_table, const int* context_lens, int max_blocks, float theta)
{
    const bool has_q = q.data() != nullptr;
    if (k.shape().size() != 4 || (has_q && (q.shape().size() != 4 || q.shape()[0] != k.shape()[0] ||
                                            q.shape()[1] != k.shape()[1] || q.shape()[3] != k.shape()[3] ||
                                            q.dtype() != k.dtype())))
        return fail("apply_rope: q must be [B, S, Hq, D] and k [B, S, Hkv, D] of one dtype");
    if (v != nullptr && (v->shape() != k.shape() || v->dtype() != k.dtype() || kc->shape().size() != 4 ||
                         vc->shape() != kc->shape() || kc->shape()[2] != k.shape()[2] ||
                         kc->shape()[3] != k.shape()[3]))
        return fail("rope_append_kv_cache: v must match k and the caches be [num_blocks, 16, Hkv, D]");
    const int rc = ffkv_rope_append(
        has_q ? q.data() : nullptr, k.data(), v ? v->data() : nullptr, code(k.dtype()), kc ? kc->data() : nullptr,
        vc ? vc->data() : nullptr, kc ? code(kc->dtype()) : code(k.dtype()), ks, vs,
        reinterpret_cast<const int32_t*>(block_table), reinterpret_cast<const int32_t*>(context_lens),
        static_cast<int>(k.shape()[0]), static_cast<int>(k.shape()[1]), has_q ? static_cast<int>(q.shape()[2]) : 0,
        static_cast<int>(k.shape()[2]), static_cast<int>(k.shape()[3]), kc ? static_cast<int>(kc->shape()[1]) : 16,
        max_blocks, kc ? static_cast<int>(kc->shape()[0]) : 0, theta, t_stream);
    report(rc, v ? "rope_append_kv_cache failed" : "apply_rope failed");
}

}  // namespace

void        set_default_stream(hipStream_t stream) { t_stream = stream; }
hipStream_t get_default_stream() { return t_stream; }
std::string last_error() { return t_error; }

void attention(Tensor& q, Tensor& k, Tensor& v, Tensor& output, void* kv_cache_block_table, int kv_head_num,
               int seq_len, int max_context_blocks, const int* context_lens)
{
    if (kv_cache_block_table == nullptr || (q.shape().size() == 4 && q.shape()[1] > 1))
        return prefill(q, k, v, nullptr, nullptr, output, kv_cache_block_table, kv_head_num, seq_len,
                       max_context_blocks, context_lens);
    decode(q, k, v, nullptr, nullptr, output, kv_cache_block_table, kv_head_num, max_context_blocks, context_lens);
}

void attention(Tensor& q, Tensor& k_cache, Tensor& v_cache, const Tensor& k_scale, const Tensor& v_scale,
               Tensor& output, void* kv_cache_block_table, int kv_head_num, int seq_len, int max_context_blocks,
               const int* context_lens)
{
    if (kv_cache_block_table == nullptr || (q.shape().size() == 4 && q.shape()[1] > 1))
        return prefill(q, k_cache, v_cache, k_scale.data_as<const float>(), v_scale.data_as<const float>(), output,
                       kv_cache_block_table, kv_head_num, seq_len, max_context_blocks, context_lens);
    decode(q, k_cache, v_cache, k_scale.data_as<const float>(), v_scale.data_as<const float>(), output,
           kv_cache_block_table, kv_head_num, max_context_blocks, context_lens);
}

void attention_shared_prefix(Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& output, void* kv_cache_block_table,
                             int kv_head_num, int max_context_blocks, const int* context_lens, int shared_blocks)
{
    if (kv_cache_block_table == nullptr || (q.shape().size() == 4 && q.shape()[1] != 1))
        return fail("attention_shared_prefix: decode only (q [B, 1, Hq, D] and a block table)");
    decode(q, k_cache, v_cache, nullptr, nullptr, output, kv_cache_block_table, kv_head_num, max_context_blocks,
           context_lens, shared_blocks);
}

void append_kv_cache_attention(const Tensor& k, const Tensor& v, Tensor& q, Tensor& k_cache, Tensor& v_cache,
                               Tensor& output, void* kv_cache_block_table, int kv_head_num, int max_context_blocks,
                               const int* context_lens)
{
    if (q.shape().size() != 4 || q.shape()[1] != 1 || k.shape().size() != 4 || k.shape()[1] != 1 ||
        v.shape() != k.shape() || k_cache.shape().size() != 4 || !is_gpu(q) || !is_gpu(k) || !is_gpu(v) ||
        !is_gpu(k_cache) || !is_gpu(v_cache) || !is_gpu(output) || kv_cache_block_table == nullptr)
        return fail("append_kv_cache_attention: decode step only (q [B, 1, Hq, D], k / v [B, 1, Hkv, D], a block "
                    "table, all tensors on the GPU)");
    const int B = static_cast<int>(q.shape()[0]);
    const int Hq = static_cast<int>(q.shape()[2]);
    const int D = static_cast<int>(q.shape()[3]);
    if (k.shape()[0] != B || k.shape()[2] != kv_head_num || k.shape()[3] != D)
        return fail("append_kv_cache_attention: k / v must be [B, 1, kv_head_num, head_dim]");
    if (output.numel() < static_cast<int64_t>(B) * Hq * D || output.dtype() != q.dtype())
        return fail("append_kv_cache_attention: output must hold B*Hq*D elements of q's dtype");
    if (k_cache.shape()[2] != kv_head_num || k_cache.shape()[3] != D || v_cache.shape() != k_cache.shape() ||
        v_cache.dtype() != k_cache.dtype())
        return fail("append_kv_cache_attention: k/v caches must both be [num_blocks, 16, kv_head_num, head_dim]");
    const size_t need = ffkv_decode_workspace_bytes(B, Hq, D, max_context_blocks, 0);
    size_t       have = 0;
    void*        ws = workspace(need, have);
    const int    rc = ffkv_append_paged_decode(
        k.data(), v.data(), code(k.dtype()), q.data(), output.data(), code(q.dtype()), k_cache.data(), v_cache.data(),
        code(k_cache.dtype()), nullptr, nullptr, reinterpret_cast<const int32_t*>(kv_cache_block_table), context_lens,
        B, Hq, kv_head_num, D, FFKV_BLOCK_SIZE, max_context_blocks, static_cast<int>(k_cache.shape()[0]), 0, 0.0f, ws,
        have, t_stream);
    report(rc, "append_kv_cache_attention failed");
}

void append_kv_cache(const Tensor& k, const Tensor& v, Tensor& k_cache, Tensor& v_cache, const int* block_table,
                     const int* context_lens, int max_blocks)
{
    append(k, v, k_cache, v_cache, nullptr, nullptr, block_table, context_lens, max_blocks);
}

void append_kv_cache(const Tensor& k, const Tensor& v, Tensor& k_cache, Tensor& v_cache, Tensor& k_scale,
                     Tensor& v_scale, const int* block_table, const int* context_lens, int max_blocks)
{
    append(k, v, k_cache, v_cache, k_scale.data_as<float>(), v_scale.data_as<float>(), block_table, context_lens,
           max_blocks);
}

void apply_rope(Tensor& q, Tensor& k, int head_dim, int seq_len, float theta, const int* context_lens)
{
    if (k.shape().size() != 4 || k.shape()[3] != head_dim || k.shape()[1] != seq_len)
        return fail("apply_rope: k must be [B, seq_len, Hkv, head_dim]");
    rope_append(q, k, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, context_lens, 0, theta);
}

void rope_append_kv_cache(Tensor& q, Tensor& k, const Tensor& v, Tensor& k_cache, Tensor& v_cache,
                          const int* block_table, const int* context_lens, int max_blocks, float theta)
{
    rope_append(q, k, &v, &k_cache, &v_cache, nullptr, nullptr, block_table, context_lens, max_blocks, theta);
}

void rope_append_kv_cache(Tensor& q, Tensor& k, const Tensor& v, Tensor& k_cache, Tensor& v_cache, Tensor& k_scale,
                          Tensor& v_scale, const int* block_table, const int* context_lens, int max_blocks,
                          float theta)
{
    rope_append(q, k, &v, &k_cache, &v_cache, k_scale.data_as<float>(), v_scale.data_as<float>(), block_table,
                context_lens, max_blocks, theta);
}

}  // namespace firefly::kernels
