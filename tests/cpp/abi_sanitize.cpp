// abi_sanitize.cpp - the C ABI's argument validation under AddressSanitizer and UBSan (tests/test_sanitize.py
// compiles firefly_amd/csrc/capi.cpp with host-side sanitizers and links it with the library's kernel objects).
//
// Every call below is rejected, or is an empty call, before any device work: invalid sizes, dtypes, block sizes,
// head_dims, group sizes, null or misaligned pointers (the pointer values are never dereferenced), workspaces too
// small, and the allocation-free decode's size limit.  Each must return its documented status code and leave a
// message (an empty one for success).
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "ffkv.h"

namespace
{

int failures = 0;

void expect(int got, int want, const char* what)
{
    const bool msg_ok = want == FFKV_OK ? ffkv_last_error()[0] == '\0' : ffkv_last_error()[0] != '\0';
    if (got != want || !msg_ok)
    {
        std::printf("FAIL %s: got %d want %d (%s)\n", what, got, want, ffkv_last_error());
        ++failures;
    }
}

void* P(uintptr_t v) { return reinterpret_cast<void*>(v); }
const int32_t* I(uintptr_t v) { return reinterpret_cast<const int32_t*>(v); }

int append(int src_dt = 2, int cache_dt = 2, int batch = 1, int seq = 1, int hkv = 8, int d = 128, int bs = 16,
           uintptr_t k = 16, uintptr_t table = 16, float* ks = nullptr)
{
    return ffkv_append(P(k), P(16), src_dt, P(16), P(16), cache_dt, ks, ks, I(table), nullptr, batch, seq, hkv, d, bs,
                       4, 4, nullptr);
}

int decode(int qo = 2, int cache = 2, int batch = 1, int hq = 32, int hkv = 8, int d = 128, int bs = 16,
           uintptr_t ctx = 16, void* ws = nullptr, size_t ws_bytes = 0, int max_blocks = 4)
{
    return ffkv_paged_decode(P(16), P(16), qo, P(16), P(16), cache, nullptr, nullptr, I(16), I(ctx), batch, hq, hkv,
                             d, bs, max_blocks, 4, 0, 0.0f, ws, ws_bytes, nullptr);
}

}  // namespace

int main()
{
    expect(append(2, 2, 1, 1, 8, 128, 32), FFKV_ERR_UNSUPPORTED, "append block_size 32");
    expect(append(2, 2, 1, 1, 8, 100), FFKV_ERR_UNSUPPORTED, "append head_dim 100 (not a multiple of 8)");
    expect(append(2, 2, 1, 1, 8, 136), FFKV_ERR_UNSUPPORTED, "append head_dim 136 (over 128, not 256)");
    expect(append(3), FFKV_ERR_UNSUPPORTED, "append int8 source");
    expect(append(2, 7), FFKV_ERR_UNSUPPORTED, "append UNKNOWN cache");
    expect(append(2, 2, -1), FFKV_ERR_INVALID_ARGUMENT, "append negative batch");
    expect(append(2, 2, 1, 1, 0), FFKV_ERR_INVALID_ARGUMENT, "append no kv heads");
    expect(append(2, 2, 1, 1, 8, 128, 16, 0), FFKV_ERR_INVALID_ARGUMENT, "append null k");
    expect(append(2, 2, 1, 1, 8, 128, 16, 16, 0), FFKV_ERR_INVALID_ARGUMENT, "append null table");
    expect(append(2, 3), FFKV_ERR_INVALID_ARGUMENT, "append int8 cache without scales");
    expect(append(2, 8), FFKV_ERR_INVALID_ARGUMENT, "append fp8 cache without scales");
    expect(append(2, 2, 1, 1, 8, 128, 16, 18), FFKV_ERR_INVALID_ARGUMENT, "append misaligned source");
    expect(append(2, 2, 0), FFKV_OK, "append empty batch");
    expect(append(2, 2, 1, 0), FFKV_OK, "append empty sequence");

    expect(decode(2, 2, 1, 32, 8, 128, 8), FFKV_ERR_UNSUPPORTED, "decode block_size 8");
    expect(decode(2, 2, 1, 32, 8, 84), FFKV_ERR_UNSUPPORTED, "decode head_dim 84 (not a multiple of 8)");
    expect(decode(2, 2, 1, 32, 8, 0), FFKV_ERR_UNSUPPORTED, "decode head_dim 0");
    expect(ffkv_paged_prefill(P(16), P(16), 2, P(16), P(16), 2, nullptr, nullptr, I(16), I(16), 1, 4, 32, 8, 96, 16,
                              4, 4, 0, 0.0f, nullptr),
           FFKV_ERR_UNSUPPORTED, "prefill head_dim 96");
    expect(decode(3), FFKV_ERR_UNSUPPORTED, "decode int8 q");
    expect(decode(2, 2, 1, 30, 8), FFKV_ERR_INVALID_ARGUMENT, "decode heads not a multiple of kv heads");
    expect(decode(2, 0, 1, 8 * 17, 8), FFKV_ERR_UNSUPPORTED, "decode group 17 on an fp32 cache");
    expect(decode(2, 2, 1, 140000, 70000), FFKV_ERR_UNSUPPORTED, "decode over 65535 heads");
    expect(decode(2, 2, 1, 32, 8, 128, 16, 0), FFKV_ERR_INVALID_ARGUMENT, "decode null context_lens");
    expect(decode(2, 3), FFKV_ERR_INVALID_ARGUMENT, "decode int8 cache without scales");
    expect(decode(2, 2, 0), FFKV_OK, "decode empty batch");
    expect(decode(2, 2, 4, 32, 8, 128, 16, 16, P(256), 4096, 600), FFKV_ERR_WORKSPACE, "decode workspace too small");
    expect(decode(2, 2, 4, 32, 8, 128, 16, 16, P(258), 1 << 30, 600), FFKV_ERR_INVALID_ARGUMENT,
           "decode misaligned workspace");

    expect(ffkv_paged_decode_noalloc(P(16), P(16), 2, P(16), P(16), 2, nullptr, nullptr, I(16), I(16), 8192, 32, 8, 128,
                                     16, 4, 4, 0, 0.0f, nullptr),
           FFKV_ERR_WORKSPACE, "noalloc decode beyond its scratch");
    expect(ffkv_paged_prefill(P(16), P(16), 2, P(16), P(16), 0, nullptr, nullptr, I(16), I(16), 1, 4, 32, 8, 128, 16,
                              4, 4, 0, 0.0f, nullptr),
           FFKV_ERR_UNSUPPORTED, "prefill fp32 cache");
    expect(ffkv_rope(P(16), P(16), 2, nullptr, 1, 1, 32, 8, 128, -1.0f, nullptr), FFKV_ERR_INVALID_ARGUMENT,
           "rope negative theta");
    std::printf("%s\n", failures == 0 ? "OK" : "FAILED");
    return failures == 0 ? 0 : 1;
}
