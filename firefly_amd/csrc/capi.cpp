// capi.cpp - the extern "C" boundary (include/ffkv.h): argument validation, split-K geometry, workspace
// handling and error reporting around the HIP launchers.
//
// The reference launches without validating anything and reports launch errors on std::cerr
// (src/kernels/attention.cu:487-491, src/model/qwen_model.cu:9-17); this layer returns a status code instead and
// keeps a per-thread message for ffkv_last_error().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "ffkv.h"
#include "ffkv_internal.h"

namespace
{

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...)
{
    char    buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok()
{
    g_last_error.clear();
    return FFKV_OK;
}

bool is_act(int dt) { return dt == FFKV_DTYPE_F32 || dt == FFKV_DTYPE_F16 || dt == FFKV_DTYPE_BF16; }
bool is_cache(int dt) { return is_act(dt) || dt == FFKV_DTYPE_I8 || dt == FFKV_DTYPE_FP8_E4M3; }
bool quantized(int dt) { return dt == FFKV_DTYPE_I8 || dt == FFKV_DTYPE_FP8_E4M3; }
// Append and decode take any head_dim that is a multiple of 8 up to 128 (as the reference's decode, one 8-element
// vector per lane of a 16-lane group: src/kernels/attention.cu:307-316), and 256; prefill and rope+append take 64,
// 128 and 256 (the reference's prefill and rope take 128, and 64 / 128).
bool head_dim_ok(int d) { return d == 256 || (d >= 8 && d <= 128 && d % 8 == 0); }
bool head_dim_mfma(int d) { return d == 64 || d == 128 || d == 256; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

int hip_fail(hipError_t e, const char* what)
{
    return fail(FFKV_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
}

int env_chunk()
{
    static const int v = []
    {
        const char* s = std::getenv("FFKV_DECODE_CHUNK");
        return s ? std::atoi(s) : 0;
    }();
    return v;
}

// FFKV_DECODE_KERNEL=generic forces the generic decode kernel (for comparisons); anything else is automatic.
bool env_force_generic()
{
    static const bool v = []
    {
        const char* s = std::getenv("FFKV_DECODE_KERNEL");
        return s && std::strcmp(s, "generic") == 0;
    }();
    return v;
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace

namespace ffkv
{

bool decode_use_mfma(int cache_dtype, int /*group*/, int head_dim)
{
    // head_dim 96 on the matrix cores too (three k-steps of 32 dims), and 80 and 112 (k-steps of 32 dims and a last
    // one of 16)
    return !env_force_generic() && cache_dtype != FFKV_DTYPE_F32 &&
           (head_dim_mfma(head_dim) || head_dim == 80 || head_dim == 96 || head_dim == 112);
}

// MFMA workspace layout: [row meta: batch x 2 int32 | (m, l): slots x num_heads x 2 fp32 | acc: slots x num_heads
// x head_dim fp32], each region 256-byte aligned, slots = items + batch (slot = work item + row) plus, in
// shared-prefix mode, prefix_chunks slots per row after those.  The public size query assumes kMfmaMaxItems items.
struct MfmaLayout
{
    int64_t meta, ml, acc, total;
};

MfmaLayout mfma_layout(int batch, int num_heads, int head_dim, int prefix_chunks = 0, int items = kMfmaMaxItems)
{
    const int64_t slots = static_cast<int64_t>(items) + batch + static_cast<int64_t>(prefix_chunks) * batch;
    MfmaLayout    l{};
    l.meta = 0;
    l.ml = align256(static_cast<int64_t>(batch) * 2 * 4);
    l.acc = l.ml + align256(slots * num_heads * 2 * 4);
    l.total = l.acc + slots * num_heads * head_dim * 4;
    return l;
}

size_t decode_mfma_workspace_bytes(int batch, int num_heads, int head_dim)
{
    return static_cast<size_t>(mfma_layout(batch, num_heads, head_dim).total);
}

// Shared-prefix split: the prefix kernel runs (kv head, chunk) groups of ceil(batch * group / 128) workgroups;
// about one workgroup per CU (256) without chunks under 8 pages (each chunk's partials cost 4 * (head_dim + 2)
// bytes per (row, head) written and read back).  FFKV_PREFIX_CHUNKS overrides the count.  The workspace's prefix
// slots are sized for this count; the fused grid (decode_pfx_plan) takes at most as many chunks.
void prefix_chunking(int batch, int group, int num_kv_heads, int shared_blocks, int& chunks, int& chunk_pages)
{
    static const int env = []
    {
        const char* s = std::getenv("FFKV_PREFIX_CHUNKS");
        return s ? std::atoi(s) : 0;
    }();
    const int64_t nrb = (static_cast<int64_t>(batch) * group + 127) / 128;
    int64_t       c = env > 0 ? env : (256 + nrb * num_kv_heads / 2) / (nrb * num_kv_heads);
    const int64_t most = env > 0 ? shared_blocks : (shared_blocks + 7) / 8;
    if (c > most) c = most;
    if (c > 256) c = 256;
    if (c < 1) c = 1;
    chunk_pages = static_cast<int>((shared_blocks + c - 1) / c);
    chunks = shared_blocks > 0 ? static_cast<int>((shared_blocks + chunk_pages - 1) / chunk_pages) : 0;
}

int decode_mfma_items(const void* kernel, int threads, int grid_y)
{
    static std::mutex                               mu;
    static std::map<std::pair<const void*, int>, int> cache;
    int                                             dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    std::lock_guard<std::mutex> lock(mu);
    auto                        key = std::make_pair(kernel, dev * 4096 + threads);
    auto                        it = cache.find(key);
    int                         resident;
    if (it != cache.end())
    {
        resident = it->second;
    }
    else
    {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu <= 0)
            per_cu = 1;
        resident = cus * per_cu;
        cache.emplace(key, resident);
    }
    int items = resident / (grid_y > 0 ? grid_y : 1);
    if (items < 1) items = 1;
    return items > kMfmaMaxItems ? kMfmaMaxItems : items;
}

int decode_cap_tokens(int max_blocks, int max_context_len)
{
    int64_t cap = static_cast<int64_t>(max_blocks) * kBlockSize;
    if (max_context_len > 0 && cap > max_context_len) cap = max_context_len;
    if (cap > (1 << 30)) cap = 1 << 30;
    return cap < 0 ? 0 : static_cast<int>(cap);
}

// Smallest chunk the workspace is sized for: at least 256 tokens and at most 64 chunks per row.
int decode_min_chunk(int cap_tokens)
{
    int64_t c = ceil_div(ceil_div(cap_tokens, 64), kBlockSize) * kBlockSize;
    return static_cast<int>(c < 256 ? 256 : c);
}

// Grow the chunk while the grid still has >= 4096 work items at the row-length bound; long chunks cost fewer
// partials, short chunks balance better.
int decode_chunk(int batch, int num_kv_heads, int cap_tokens)
{
    const int min_chunk = decode_min_chunk(cap_tokens);
    int       chunk = min_chunk;
    if (env_chunk() > 0)
    {
        chunk = static_cast<int>(ceil_div(env_chunk(), kBlockSize) * kBlockSize);
        return chunk < min_chunk ? min_chunk : chunk;
    }
    const int64_t pairs = static_cast<int64_t>(batch) * num_kv_heads;
    while (chunk < 4096 && pairs * ceil_div(cap_tokens, 2 * chunk) >= 4096) chunk *= 2;
    return chunk;
}

size_t decode_workspace_bytes(int batch, int num_heads, int head_dim, int cap_tokens)
{
    const int64_t chunks = ceil_div(cap_tokens, decode_min_chunk(cap_tokens));
    if (chunks <= 1) return 0;
    const int64_t parts = static_cast<int64_t>(batch) * num_heads * chunks;
    const int64_t ml = ceil_div(parts * 2 * 4, 256) * 256;
    return static_cast<size_t>(ml + parts * head_dim * 4);
}

}  // namespace ffkv

extern "C" {

const char* ffkv_last_error(void) { return g_last_error.c_str(); }

const char* ffkv_version(void) { return "ffkv 0.1.0 gfx950"; }

int ffkv_append(const void* k_src, const void* v_src, int src_dtype, void* k_cache, void* v_cache, int cache_dtype,
                float* k_scale, float* v_scale, const int32_t* block_table, const int32_t* context_lens, int batch,
                int seq_len, int num_kv_heads, int head_dim, int block_size, int max_blocks, int num_blocks,
                void* stream)
{
    if (block_size != FFKV_BLOCK_SIZE) return fail(FFKV_ERR_UNSUPPORTED, "block_size must be 16, got %d", block_size);
    if (!is_act(src_dtype)) return fail(FFKV_ERR_UNSUPPORTED, "unsupported source dtype %d", src_dtype);
    if (!is_cache(cache_dtype)) return fail(FFKV_ERR_UNSUPPORTED, "unsupported cache dtype %d", cache_dtype);
    if (!head_dim_ok(head_dim))
        return fail(FFKV_ERR_UNSUPPORTED, "head_dim must be a multiple of 8 up to 128, or 256, got %d", head_dim);
    if (batch < 0 || seq_len < 0 || num_kv_heads <= 0 || max_blocks < 0 || num_blocks < 0)
        return fail(FFKV_ERR_INVALID_ARGUMENT, "negative size (batch %d seq_len %d kv_heads %d max_blocks %d "
                    "num_blocks %d)", batch, seq_len, num_kv_heads, max_blocks, num_blocks);
    if (batch == 0 || seq_len == 0) return ok();
    if (!k_src || !v_src || !k_cache || !v_cache || !block_table)
        return fail(FFKV_ERR_INVALID_ARGUMENT, "null source, cache or block_table pointer");
    if (quantized(cache_dtype) && (!k_scale || !v_scale))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "quantized cache needs k_scale and v_scale");
    if (!aligned16(k_src) || !aligned16(v_src) || !aligned16(k_cache) || !aligned16(v_cache))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "source and cache pointers must be 16-byte aligned");

    ffkv::AppendArgs a{k_src,      v_src,        k_cache,   v_cache,     k_scale,  v_scale,
                       block_table, context_lens, src_dtype, cache_dtype, batch,    seq_len,
                       num_kv_heads, head_dim,    max_blocks, num_blocks};
    hipError_t e = ffkv::launch_append(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "append launch");
    return ok();
}

int ffkv_paged_prefill(const void* q, void* out, int qo_dtype, const void* k_cache, const void* v_cache,
                       int cache_dtype, const float* k_scale, const float* v_scale, const int32_t* block_table,
                       const int32_t* context_lens, int batch, int seq_len, int num_heads, int num_kv_heads,
                       int head_dim, int block_size, int max_blocks, int num_blocks, int max_context_len, float scale,
                       void* stream)
{
    const bool paged = block_table != nullptr;
    if (block_size != FFKV_BLOCK_SIZE) return fail(FFKV_ERR_UNSUPPORTED, "block_size must be 16, got %d", block_size);
    if (!is_act(qo_dtype)) return fail(FFKV_ERR_UNSUPPORTED, "unsupported q/out dtype %d", qo_dtype);
    if (!is_cache(cache_dtype) || cache_dtype == FFKV_DTYPE_F32)
        return fail(FFKV_ERR_UNSUPPORTED, "prefill supports F16, BF16, I8 and FP8_E4M3 caches, got dtype %d",
                    cache_dtype);
    if (!head_dim_mfma(head_dim)) return fail(FFKV_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256, got %d", head_dim);
    if (batch < 0 || seq_len < 0 || num_heads <= 0 || num_kv_heads <= 0 || (paged && (max_blocks < 0 || num_blocks < 0)))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "bad size (batch %d seq_len %d heads %d kv_heads %d max_blocks %d "
                    "num_blocks %d)", batch, seq_len, num_heads, num_kv_heads, max_blocks, num_blocks);
    if (num_heads % num_kv_heads != 0)
        return fail(FFKV_ERR_INVALID_ARGUMENT, "num_heads %d is not a multiple of num_kv_heads %d", num_heads,
                    num_kv_heads);
    if (batch > 65535 || num_kv_heads > 65535)
        return fail(FFKV_ERR_UNSUPPORTED, "batch and num_kv_heads must be <= 65535");
    if (static_cast<int64_t>(seq_len) * (num_heads / num_kv_heads) > INT32_MAX - 64)
        return fail(FFKV_ERR_UNSUPPORTED, "seq_len * group too large");
    if (static_cast<int64_t>(batch) * num_kv_heads *
            ((static_cast<int64_t>(seq_len) * (num_heads / num_kv_heads) + 127) / 128) > INT32_MAX - 64 * 1024)
        return fail(FFKV_ERR_UNSUPPORTED, "batch * num_kv_heads * ceil(seq_len * group / 128) too large");
    if (batch == 0 || seq_len == 0) return ok();
    if (!q || !out || !k_cache || !v_cache || (paged && !context_lens))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "null q, out, cache or context_lens pointer");
    if (!paged && cache_dtype == FFKV_DTYPE_I8)
        return fail(FFKV_ERR_UNSUPPORTED, "int8 K/V need a block table (their scales are per page slot)");
    if (quantized(cache_dtype) && (!k_scale || !v_scale))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "quantized cache needs k_scale and v_scale");
    if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "q, out and cache pointers must be 16-byte aligned");

    const float       sm_scale = scale > 0.0f ? scale : 1.0f / sqrtf(static_cast<float>(head_dim));
    ffkv::PrefillArgs a{};
    a.q = q;
    a.out = out;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.block_table = block_table;
    a.context_lens = context_lens;
    a.qo_dtype = qo_dtype;
    a.cache_dtype = cache_dtype;
    a.batch = batch;
    a.seq_len = seq_len;
    a.num_heads = num_heads;
    a.num_kv_heads = num_kv_heads;
    a.group = num_heads / num_kv_heads;
    a.head_dim = head_dim;
    a.max_blocks = paged ? max_blocks : 0;
    a.num_blocks = paged ? num_blocks : 0;
    a.cap_tokens = paged ? ffkv::decode_cap_tokens(max_blocks, max_context_len) : seq_len;
    a.paged = paged;
    a.scale_log2 = sm_scale * 1.4426950408889634f;
    hipError_t e = ffkv::launch_prefill(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "prefill launch");
    return ok();
}

int ffkv_rope(void* q, void* k, int dtype, const int32_t* context_lens, int batch, int seq_len, int num_heads,
              int num_kv_heads, int head_dim, float rope_theta, void* stream)
{
    return ffkv_rope_append(q, k, nullptr, dtype, nullptr, nullptr, dtype, nullptr, nullptr, nullptr, context_lens,
                            batch, seq_len, num_heads, num_kv_heads, head_dim, FFKV_BLOCK_SIZE, 0, 0, rope_theta,
                            stream);
}

int ffkv_rope_append(void* q, void* k, const void* v, int src_dtype, void* k_cache, void* v_cache, int cache_dtype,
                     float* k_scale, float* v_scale, const int32_t* block_table, const int32_t* context_lens,
                     int batch, int seq_len, int num_heads, int num_kv_heads, int head_dim, int block_size,
                     int max_blocks, int num_blocks, float rope_theta, void* stream)
{
    const bool append = k_cache != nullptr || v_cache != nullptr;
    if (block_size != FFKV_BLOCK_SIZE) return fail(FFKV_ERR_UNSUPPORTED, "block_size must be 16, got %d", block_size);
    if (!is_act(src_dtype)) return fail(FFKV_ERR_UNSUPPORTED, "unsupported q/k/v dtype %d", src_dtype);
    if (append && !is_cache(cache_dtype)) return fail(FFKV_ERR_UNSUPPORTED, "unsupported cache dtype %d", cache_dtype);
    if (!head_dim_mfma(head_dim)) return fail(FFKV_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256, got %d", head_dim);
    if (q == nullptr) num_heads = 0;
    if (batch < 0 || seq_len < 0 || num_heads < 0 || num_kv_heads <= 0 || max_blocks < 0 || num_blocks < 0)
        return fail(FFKV_ERR_INVALID_ARGUMENT, "negative size (batch %d seq_len %d heads %d kv_heads %d max_blocks %d "
                    "num_blocks %d)", batch, seq_len, num_heads, num_kv_heads, max_blocks, num_blocks);
    if (!(rope_theta > 0.0f) || rope_theta == __builtin_huge_valf())
        return fail(FFKV_ERR_INVALID_ARGUMENT, "rope_theta must be positive and finite, got %g",
                    static_cast<double>(rope_theta));
    if (batch == 0 || seq_len == 0) return ok();
    if (!k) return fail(FFKV_ERR_INVALID_ARGUMENT, "null k pointer");
    if (append && (!v || !k_cache || !v_cache || !block_table))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "null v, cache or block_table pointer");
    if (append && quantized(cache_dtype) && (!k_scale || !v_scale))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "quantized cache needs k_scale and v_scale");
    if ((q && !aligned16(q)) || !aligned16(k) || (append && (!aligned16(v) || !aligned16(k_cache) ||
                                                             !aligned16(v_cache))))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "q, k, v and cache pointers must be 16-byte aligned");

    ffkv::RopeArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.k_cache = append ? k_cache : nullptr;
    a.v_cache = append ? v_cache : nullptr;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.block_table = block_table;
    a.context_lens = context_lens;
    a.src_dtype = src_dtype;
    a.cache_dtype = cache_dtype;
    a.batch = batch;
    a.seq_len = seq_len;
    a.num_heads = num_heads;
    a.num_kv_heads = num_kv_heads;
    a.head_dim = head_dim;
    a.max_blocks = max_blocks;
    a.num_blocks = num_blocks;
    a.theta = rope_theta;
    hipError_t e = ffkv::launch_rope_append(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, append ? "rope_append launch" : "rope launch");
    return ok();
}

size_t ffkv_kv_block_bytes(int cache_dtype, int num_kv_heads, int head_dim)
{
    if (num_kv_heads <= 0 || head_dim <= 0) return 0;
    const size_t rows = static_cast<size_t>(FFKV_BLOCK_SIZE) * static_cast<size_t>(num_kv_heads);  // token x head
    const size_t d = static_cast<size_t>(head_dim);
    switch (cache_dtype)
    {
        case FFKV_DTYPE_F32:
            return rows * d * 4 * 2;
        case FFKV_DTYPE_F16:
        case FFKV_DTYPE_BF16:
            return rows * d * 2 * 2;
        case FFKV_DTYPE_I8:
            return rows * (d + 4) * 2;  // codes + one fp32 scale per (token, head), K and V
        case FFKV_DTYPE_FP8_E4M3:
            return rows * d * 2;
        default:
            return 0;
    }
}

size_t ffkv_decode_workspace_bytes(int batch, int num_heads, int head_dim, int max_blocks, int max_context_len)
{
    if (batch <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
    const size_t generic = ffkv::decode_workspace_bytes(batch, num_heads, head_dim,
                                                        ffkv::decode_cap_tokens(max_blocks, max_context_len));
    const size_t mfma = ffkv::decode_mfma_workspace_bytes(batch, num_heads, head_dim);
    return generic > mfma ? generic : mfma;
}

namespace
{

// Split-K scratch of ffkv_paged_decode_noalloc: a file-scope device array, one copy on every GPU the library runs
// on, held until the process ends.  Host code never passes `scratch` itself to a kernel (on the host it names a
// stand-in, not device memory): scratch_for_device() resolves the current device's copy once with
// hipGetSymbolAddress and every later use goes through that address.  Calls on one GPU share its copy; the
// kernels write every partial before reading it, so nothing needs clearing between calls, but calls that overlap
// in time on one GPU race.
__device__ __align__(256) static unsigned char scratch[FFKV_NOALLOC_SCRATCH_BYTES];

std::mutex         g_scratch_mu;
std::map<int, void*> g_scratch;  // device -> address of its copy of `scratch`

int scratch_for_device(void** ptr)
{
    int        dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto                        it = g_scratch.find(dev);
    if (it == g_scratch.end())
    {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        it = g_scratch.emplace(dev, p).first;
    }
    *ptr = it->second;
    return FFKV_OK;
}

// workspace == kNoAlloc: the decode uses this library's static scratch (ffkv_paged_decode_noalloc) and allocates
// nothing; sizes whose partials do not fit it are rejected.
void* const kNoAlloc = reinterpret_cast<void*>(~uintptr_t{0});

int decode_impl(const void* q, void* out, int qo_dtype, const void* k_cache, const void* v_cache, int cache_dtype,
                const float* k_scale, const float* v_scale, const int32_t* block_table, const int32_t* context_lens,
                int batch, int num_heads, int num_kv_heads, int head_dim, int block_size, int max_blocks,
                int num_blocks, int max_context_len, float scale, int shared_blocks, void* workspace,
                size_t workspace_bytes, void* stream, const void* k_new = nullptr, const void* v_new = nullptr)
{
    if (block_size != FFKV_BLOCK_SIZE) return fail(FFKV_ERR_UNSUPPORTED, "block_size must be 16, got %d", block_size);
    if (!is_act(qo_dtype)) return fail(FFKV_ERR_UNSUPPORTED, "unsupported q/out dtype %d", qo_dtype);
    if (!is_cache(cache_dtype)) return fail(FFKV_ERR_UNSUPPORTED, "unsupported cache dtype %d", cache_dtype);
    if (!head_dim_ok(head_dim))
        return fail(FFKV_ERR_UNSUPPORTED, "head_dim must be a multiple of 8 up to 128, or 256, got %d", head_dim);
    if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || max_blocks < 0 || num_blocks < 0)
        return fail(FFKV_ERR_INVALID_ARGUMENT, "bad size (batch %d heads %d kv_heads %d max_blocks %d num_blocks %d)",
                    batch, num_heads, num_kv_heads, max_blocks, num_blocks);
    if (num_heads % num_kv_heads != 0)
        return fail(FFKV_ERR_INVALID_ARGUMENT, "num_heads %d is not a multiple of num_kv_heads %d", num_heads,
                    num_kv_heads);
    const int group = num_heads / num_kv_heads;
    // the matrix-core decode takes any group (one wave per block of 16 query heads); the fp32-cache kernel 16 at most
    if (group > 16 && !ffkv::decode_use_mfma(cache_dtype, group, head_dim))
        return fail(FFKV_ERR_UNSUPPORTED, "GQA group size %d exceeds 16 (fp32 caches, or the generic decode forced)",
                    group);
    if (batch > 65535 || num_heads > 65535)
        return fail(FFKV_ERR_UNSUPPORTED, "batch and num_heads must be <= 65535");
    if (batch == 0) return ok();
    if (!q || !out || !k_cache || !v_cache || !block_table || !context_lens)
        return fail(FFKV_ERR_INVALID_ARGUMENT, "null q, out, cache, block_table or context_lens pointer");
    if (quantized(cache_dtype) && (!k_scale || !v_scale))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "quantized cache needs k_scale and v_scale");
    if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "q, out and cache pointers must be 16-byte aligned");

    const int cap = ffkv::decode_cap_tokens(max_blocks, max_context_len);
    if (static_cast<int64_t>(batch) * ceil_div(cap, FFKV_BLOCK_SIZE) > INT32_MAX)
        return fail(FFKV_ERR_UNSUPPORTED, "batch * pages per row exceeds 2^31 - 1 (batch %d, %d tokens per row)",
                    batch, cap);
    if (shared_blocks < 0 || shared_blocks > max_blocks)
        return fail(FFKV_ERR_INVALID_ARGUMENT, "shared_blocks %d outside 0 .. max_blocks %d", shared_blocks,
                    max_blocks);
    const bool mfma = ffkv::decode_use_mfma(cache_dtype, group, head_dim);
    // shared-prefix split: matrix-core decode (16- and 8-bit caches; fp32 caches take the plain decode, same results)
    const int skip = mfma && head_dim_mfma(head_dim)  // the prefix partials' kernel takes 64, 128 and 256
                         ? std::min(shared_blocks, static_cast<int>(ceil_div(cap, FFKV_BLOCK_SIZE)))
                         : 0;
    int pfx_chunks = 0, pfx_chunk_pages = 0;
    if (skip > 0) ffkv::prefix_chunking(batch, group, num_kv_heads, skip, pfx_chunks, pfx_chunk_pages);
    const int  chunk = ffkv::decode_chunk(batch, num_kv_heads, cap);
    const int  max_chunks = static_cast<int>(ceil_div(cap > 0 ? cap : 1, chunk));

    ffkv::DecodeArgs a{};
    a.qo_dtype = qo_dtype;
    a.cache_dtype = cache_dtype;
    a.batch = batch;
    a.num_heads = num_heads;
    a.num_kv_heads = num_kv_heads;
    a.group = group;
    a.head_dim = head_dim;
    // shared prefix on 16-bit pages at head_dim 128: the prefix partials run inside the decode's grid
    ffkv::DecodePfxPlan plan{};
    const bool          fused_pfx = skip > 0 && ffkv::decode_pfx_plan(a, skip, pfx_chunks, plan);
    if (fused_pfx)
    {
        pfx_chunks = plan.chunks;
        pfx_chunk_pages = plan.chunk_pages;
        a.pfx_items = plan.pfx_items;
        a.pfx_share = plan.pfx_share;
    }
    a.items = fused_pfx ? plan.items : (mfma ? ffkv::decode_mfma_launch_items(a) : 0);

    // workspace layout: MFMA kernel see mfma_layout, generic kernel [ml | acc] (none for single-chunk rows)
    ffkv::MfmaLayout lay{};
    int64_t          need = 0;
    if (mfma)
    {
        lay = ffkv::mfma_layout(batch, num_heads, head_dim, pfx_chunks, a.items);
        need = lay.total;
    }
    else if (max_chunks > 1)
    {
        const int64_t parts = static_cast<int64_t>(batch) * num_heads * max_chunks;
        lay.ml = 0;
        lay.acc = align256(parts * 2 * 4);
        need = lay.acc + parts * head_dim * 4;
    }

    hipStream_t s = static_cast<hipStream_t>(stream);
    void*       ws = workspace;
    bool        owned = false;
    if (ws == kNoAlloc)
    {
        if (need > static_cast<int64_t>(FFKV_NOALLOC_SCRATCH_BYTES))
            return fail(FFKV_ERR_WORKSPACE,
                        "ffkv_paged_decode_noalloc: these sizes need %lld bytes of split-K scratch, more than its "
                        "maximum of %lld bytes (use ffkv_paged_decode with a workspace)",
                        static_cast<long long>(need), static_cast<long long>(FFKV_NOALLOC_SCRATCH_BYTES));
        if (const int rc = scratch_for_device(&ws)) return rc;
        workspace_bytes = FFKV_NOALLOC_SCRATCH_BYTES;
    }
    if (need > 0)
    {
        if (ws == nullptr)
        {
            hipError_t e = hipMallocAsync(&ws, static_cast<size_t>(need), s);
            if (e != hipSuccess) return hip_fail(e, "decode workspace hipMallocAsync");
            owned = true;
        }
        else if (workspace_bytes < static_cast<size_t>(need))
        {
            return fail(FFKV_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %lld bytes needed",
                        workspace_bytes, static_cast<long long>(need));
        }
        else if (!aligned16(ws))
        {
            return fail(FFKV_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
        }
    }
    char* wsb = static_cast<char*>(ws);

    const float sm_scale = scale > 0.0f ? scale : 1.0f / sqrtf(static_cast<float>(head_dim));
    a.q = q;
    a.out = out;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.block_table = block_table;
    a.context_lens = context_lens;
    a.ws_meta = need > 0 && mfma ? reinterpret_cast<int32_t*>(wsb + lay.meta) : nullptr;
    a.ws_ml = need > 0 ? reinterpret_cast<float*>(wsb + lay.ml) : nullptr;
    a.ws_acc = need > 0 ? reinterpret_cast<float*>(wsb + lay.acc) : nullptr;
    a.max_blocks = max_blocks;
    a.num_blocks = num_blocks;
    a.cap_tokens = cap;
    a.chunk = chunk;
    a.max_chunks = max_chunks;
    a.scale_log2 = sm_scale * 1.4426950408889634f;
    hipError_t        e = hipSuccess;
    ffkv::PrefillArgs p{};
    if (skip > 0)
    {
        a.skip_blocks = skip;
        a.pfx_chunks = pfx_chunks;
        a.pfx_slot0 = a.items + batch;
        p.q = q;
        p.k_cache = k_cache;
        p.v_cache = v_cache;
        p.k_scale = k_scale;
        p.v_scale = v_scale;
        p.block_table = block_table;
        p.context_lens = context_lens;
        p.qo_dtype = qo_dtype;
        p.cache_dtype = cache_dtype;
        p.batch = batch;
        p.seq_len = 1;
        p.num_heads = num_heads;
        p.num_kv_heads = num_kv_heads;
        p.group = group;
        p.head_dim = head_dim;
        p.max_blocks = max_blocks;
        p.num_blocks = num_blocks;
        p.cap_tokens = cap;
        p.paged = true;
        p.scale_log2 = a.scale_log2;
        p.pfx_blocks = skip;
        p.pfx_chunks = pfx_chunks;
        p.pfx_chunk_pages = pfx_chunk_pages;
        p.pfx_slot0 = a.pfx_slot0;
        p.ws_ml = a.ws_ml;
        p.ws_acc = a.ws_acc;
        if (!fused_pfx) e = ffkv::launch_prefix_partials(p, s);
    }
    if (k_new != nullptr && e == hipSuccess)
    {
        if (mfma && skip == 0)
        {
            a.k_new = k_new;  // the decode kernel writes the step's token into its page and attends it
            a.v_new = v_new;
        }
        else
        {
            ffkv::AppendArgs ap{k_new,        v_new,        const_cast<void*>(k_cache), const_cast<void*>(v_cache),
                                const_cast<float*>(k_scale), const_cast<float*>(v_scale), block_table,
                                context_lens, cache_dtype,  cache_dtype,  batch, 1, num_kv_heads, head_dim,
                                max_blocks,   num_blocks};
            e = ffkv::launch_append(ap, s);
        }
    }
    if (e == hipSuccess)
        e = fused_pfx ? ffkv::launch_decode_pfx(a, p, plan.gy, s)
                      : (mfma ? ffkv::launch_decode_mfma(a, s) : ffkv::launch_decode(a, s));
    if (owned)
    {
        hipError_t fe = hipFreeAsync(ws, s);
        if (e == hipSuccess) e = fe;
    }
    if (e != hipSuccess) return hip_fail(e, "decode launch");
    return ok();
}

}  // namespace

int ffkv_paged_decode(const void* q, void* out, int qo_dtype, const void* k_cache, const void* v_cache,
                      int cache_dtype, const float* k_scale, const float* v_scale, const int32_t* block_table,
                      const int32_t* context_lens, int batch, int num_heads, int num_kv_heads, int head_dim,
                      int block_size, int max_blocks, int num_blocks, int max_context_len, float scale,
                      void* workspace, size_t workspace_bytes, void* stream)
{
    return decode_impl(q, out, qo_dtype, k_cache, v_cache, cache_dtype, k_scale, v_scale, block_table, context_lens,
                       batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks, num_blocks, max_context_len,
                       scale, 0, workspace, workspace_bytes, stream);
}

int ffkv_paged_decode_noalloc(const void* q, void* out, int qo_dtype, const void* k_cache, const void* v_cache,
                              int cache_dtype, const float* k_scale, const float* v_scale, const int32_t* block_table,
                              const int32_t* context_lens, int batch, int num_heads, int num_kv_heads, int head_dim,
                              int block_size, int max_blocks, int num_blocks, int max_context_len, float scale,
                              void* stream)
{
    return decode_impl(q, out, qo_dtype, k_cache, v_cache, cache_dtype, k_scale, v_scale, block_table, context_lens,
                       batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks, num_blocks, max_context_len,
                       scale, 0, kNoAlloc, 0, stream);
}

int ffkv_append_paged_decode(const void* k_new, const void* v_new, int src_dtype, const void* q, void* out,
                             int qo_dtype, void* k_cache, void* v_cache, int cache_dtype, float* k_scale,
                             float* v_scale, const int32_t* block_table, const int32_t* context_lens, int batch,
                             int num_heads, int num_kv_heads, int head_dim, int block_size, int max_blocks,
                             int num_blocks, int max_context_len, float scale, void* workspace,
                             size_t workspace_bytes, void* stream)
{
    if (!is_act(src_dtype)) return fail(FFKV_ERR_UNSUPPORTED, "unsupported source dtype %d", src_dtype);
    if (batch > 0 && (!k_new || !v_new)) return fail(FFKV_ERR_INVALID_ARGUMENT, "null k_new or v_new pointer");
    if (batch > 0 && (!aligned16(k_new) || !aligned16(v_new)))
        return fail(FFKV_ERR_INVALID_ARGUMENT, "k_new and v_new must be 16-byte aligned");
    // One launch when the step's k/v already have the cache's 16-bit type; otherwise the append kernel, then the
    // decode.
    const bool fused = src_dtype == cache_dtype && (cache_dtype == FFKV_DTYPE_BF16 || cache_dtype == FFKV_DTYPE_F16);
    if (!fused)
    {
        const int rc = ffkv_append(k_new, v_new, src_dtype, k_cache, v_cache, cache_dtype, k_scale, v_scale,
                                   block_table, context_lens, batch, 1, num_kv_heads, head_dim, block_size,
                                   max_blocks, num_blocks, stream);
        if (rc != FFKV_OK) return rc;
        return ffkv_paged_decode(q, out, qo_dtype, k_cache, v_cache, cache_dtype, k_scale, v_scale, block_table,
                                 context_lens, batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks,
                                 num_blocks, max_context_len, scale, workspace, workspace_bytes, stream);
    }
    return decode_impl(q, out, qo_dtype, k_cache, v_cache, cache_dtype, k_scale, v_scale, block_table, context_lens,
                       batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks, num_blocks, max_context_len,
                       scale, 0, workspace, workspace_bytes, stream, k_new, v_new);
}

size_t ffkv_decode_shared_prefix_workspace_bytes(int batch, int num_heads, int num_kv_heads, int head_dim,
                                                 int max_blocks, int max_context_len, int shared_blocks)
{
    if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
    const size_t plain = ffkv_decode_workspace_bytes(batch, num_heads, head_dim, max_blocks, max_context_len);
    const int    cap = ffkv::decode_cap_tokens(max_blocks, max_context_len);
    const int    skip = std::min(std::max(shared_blocks, 0), static_cast<int>(ceil_div(cap, FFKV_BLOCK_SIZE)));
    int          chunks = 0, chunk_pages = 0;
    if (skip > 0) ffkv::prefix_chunking(batch, num_heads / num_kv_heads, num_kv_heads, skip, chunks, chunk_pages);
    const size_t shared = static_cast<size_t>(ffkv::mfma_layout(batch, num_heads, head_dim, chunks).total);
    return plain > shared ? plain : shared;
}

int ffkv_paged_decode_shared_prefix(const void* q, void* out, int qo_dtype, const void* k_cache, const void* v_cache,
                                    int cache_dtype, const float* k_scale, const float* v_scale,
                                    const int32_t* block_table, const int32_t* context_lens, int batch, int num_heads,
                                    int num_kv_heads, int head_dim, int block_size, int max_blocks, int num_blocks,
                                    int max_context_len, float scale, int shared_blocks, void* workspace,
                                    size_t workspace_bytes, void* stream)
{
    return decode_impl(q, out, qo_dtype, k_cache, v_cache, cache_dtype, k_scale, v_scale, block_table, context_lens,
                       batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks, num_blocks, max_context_len,
                       scale, shared_blocks, workspace, workspace_bytes, stream);
}

}  // extern "C"
