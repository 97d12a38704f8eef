// kernels_api_shim.cpp - C entry points over the firefly:: C++ API, for tests/test_gpu_cxx_api.py.
//
// Wraps caller device buffers in non-owning firefly::Tensor views and calls the drop-in operators exactly as the
// reference's model does (src/model/qwen_model.cu:138-156): kernels::append_kv_cache, then kernels::attention on
// the paged caches with the block table and context_lens device pointers.  Returns 0 or -1 with the error text
// from kernels::last_error().
#include <cstring>
#include <string>
#include <vector>

#include "firefly/kernels.h"

using namespace firefly;

extern "C" {

static thread_local std::string g_err;

const char* kas_last_error() { return g_err.c_str(); }

// kernels::release_workspace on the calling thread's workspace for `stream`.
int kas_release_workspace(void* stream)
{
    kernels::release_workspace(static_cast<hipStream_t>(stream));
    if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
    return 0;
}

// q [B,1,Hq,D], k_new/v_new [B,S,Hkv,D] in dtype qd; caches [N,16,Hkv,D] in dtype cd; out [B,1,Hq*D] in dtype qd.
int kas_append_then_decode(void* q, void* k_new, void* v_new, void* k_cache, void* v_cache, void* k_scale,
                           void* v_scale, int scale_rows, void* out, const int* block_table, const int* context_lens,
                           int B, int S, int Hq, int Hkv, int D, int N, int max_blocks, int qd, int cd, void* stream)
{
    kernels::set_default_stream(static_cast<hipStream_t>(stream));
    const DType qt = static_cast<DType>(qd), ct = static_cast<DType>(cd);
    Tensor      tq = Tensor::from_external(q, {B, 1, Hq, D}, qt, Device::GPU);
    Tensor      tk = Tensor::from_external(k_new, {B, S, Hkv, D}, qt, Device::GPU);
    Tensor      tv = Tensor::from_external(v_new, {B, S, Hkv, D}, qt, Device::GPU);
    Tensor      kc = Tensor::from_external(k_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    Tensor      vc = Tensor::from_external(v_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    Tensor      to = Tensor::from_external(out, {B, 1, Hq * D}, qt, Device::GPU);
    const bool  quant = ct == DType::I8 || ct == DType::FP8_E4M3;
    if (quant)
    {
        std::vector<int64_t> sshape = ct == DType::I8 ? std::vector<int64_t>{N, 16, Hkv} : std::vector<int64_t>{Hkv};
        (void)scale_rows;
        Tensor ks = Tensor::from_external(k_scale, sshape, DType::F32, Device::GPU);
        Tensor vs = Tensor::from_external(v_scale, sshape, DType::F32, Device::GPU);
        kernels::append_kv_cache(tk, tv, kc, vc, ks, vs, block_table, context_lens, max_blocks);
        if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
        kernels::attention(tq, kc, vc, ks, vs, to, const_cast<int*>(block_table), Hkv, 1, max_blocks, context_lens);
    }
    else
    {
        kernels::append_kv_cache(tk, tv, kc, vc, block_table, context_lens, max_blocks);
        if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
        kernels::attention(tq, kc, vc, to, const_cast<int*>(block_table), Hkv, 1, max_blocks, context_lens);
    }
    if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
    return 0;
}

// kernels::attention_shared_prefix over 16-bit caches already holding the step's tokens: q [B,1,Hq,D] (dtype qd),
// caches [N,16,Hkv,D] (dtype cd), out [B,1,Hq*D].
int kas_decode_shared_prefix(void* q, void* k_cache, void* v_cache, void* out, const int* block_table,
                             const int* context_lens, int B, int Hq, int Hkv, int D, int N, int max_blocks, int qd,
                             int cd, int shared_blocks, void* stream)
{
    kernels::set_default_stream(static_cast<hipStream_t>(stream));
    const DType qt = static_cast<DType>(qd), ct = static_cast<DType>(cd);
    Tensor      tq = Tensor::from_external(q, {B, 1, Hq, D}, qt, Device::GPU);
    Tensor      kc = Tensor::from_external(k_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    Tensor      vc = Tensor::from_external(v_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    Tensor      to = Tensor::from_external(out, {B, 1, Hq * D}, qt, Device::GPU);
    kernels::attention_shared_prefix(tq, kc, vc, to, const_cast<int*>(block_table), Hkv, max_blocks, context_lens,
                                     shared_blocks);
    if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
    return 0;
}

// The decode step as one call: kernels::append_kv_cache_attention(k_new, v_new, q, ...), k_new / v_new
// [B, 1, Hkv, D] in dtype kd, q / out in dtype qd, caches [N, 16, Hkv, D] in dtype cd.
int kas_append_attention(void* k_new, void* v_new, int kd, void* q, void* k_cache, void* v_cache, void* out,
                         const int* block_table, const int* context_lens, int B, int Hq, int Hkv, int D, int N,
                         int max_blocks, int qd, int cd, void* stream)
{
    kernels::set_default_stream(static_cast<hipStream_t>(stream));
    const DType qt = static_cast<DType>(qd), ct = static_cast<DType>(cd), kt = static_cast<DType>(kd);
    Tensor      tk = Tensor::from_external(k_new, {B, 1, Hkv, D}, kt, Device::GPU);
    Tensor      tv = Tensor::from_external(v_new, {B, 1, Hkv, D}, kt, Device::GPU);
    Tensor      tq = Tensor::from_external(q, {B, 1, Hq, D}, qt, Device::GPU);
    Tensor      kc = Tensor::from_external(k_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    Tensor      vc = Tensor::from_external(v_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    Tensor      to = Tensor::from_external(out, {B, 1, Hq * D}, qt, Device::GPU);
    kernels::append_kv_cache_attention(tk, tv, tq, kc, vc, to, const_cast<int*>(block_table), Hkv, max_blocks,
                                       context_lens);
    if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
    return 0;
}

// The reference's per-layer sequence with the rotary embedding (src/model/qwen_model.cu:136-143): fused == 1
// calls kernels::rope_append_kv_cache, else kernels::apply_rope then kernels::append_kv_cache.  q [B,S,Hq,D],
// k/v [B,S,Hkv,D] in dtype qd (q and k rotated in place); caches [N,16,Hkv,D] in dtype cd.
int kas_rope_append(void* q, void* k_new, void* v_new, void* k_cache, void* v_cache, void* k_scale, void* v_scale,
                    const int* block_table, const int* context_lens, int B, int S, int Hq, int Hkv, int D, int N,
                    int max_blocks, int qd, int cd, float theta, int fused, void* stream)
{
    kernels::set_default_stream(static_cast<hipStream_t>(stream));
    const DType qt = static_cast<DType>(qd), ct = static_cast<DType>(cd);
    Tensor      tq = Tensor::from_external(q, {B, S, Hq, D}, qt, Device::GPU);
    Tensor      tk = Tensor::from_external(k_new, {B, S, Hkv, D}, qt, Device::GPU);
    Tensor      tv = Tensor::from_external(v_new, {B, S, Hkv, D}, qt, Device::GPU);
    Tensor      kc = Tensor::from_external(k_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    Tensor      vc = Tensor::from_external(v_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    const bool  quant = ct == DType::I8 || ct == DType::FP8_E4M3;
    std::vector<int64_t> sshape = ct == DType::I8 ? std::vector<int64_t>{N, 16, Hkv} : std::vector<int64_t>{Hkv};
    Tensor      ks = Tensor::from_external(k_scale, sshape, DType::F32, Device::GPU);
    Tensor      vs = Tensor::from_external(v_scale, sshape, DType::F32, Device::GPU);
    if (fused)
    {
        if (quant)
            kernels::rope_append_kv_cache(tq, tk, tv, kc, vc, ks, vs, block_table, context_lens, max_blocks, theta);
        else
            kernels::rope_append_kv_cache(tq, tk, tv, kc, vc, block_table, context_lens, max_blocks, theta);
    }
    else
    {
        kernels::apply_rope(tq, tk, D, S, theta, context_lens);
        if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
        if (quant)
            kernels::append_kv_cache(tk, tv, kc, vc, ks, vs, block_table, context_lens, max_blocks);
        else
            kernels::append_kv_cache(tk, tv, kc, vc, block_table, context_lens, max_blocks);
    }
    if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
    return 0;
}

// The reference's prefill branch: kernels::attention(q, k, v, out, nullptr, Hkv, S, max_blocks, nullptr) with the
// chunk's contiguous q [B,S,Hq,D], k/v [B,S,Hkv,D] (src/model/qwen_model.cu:147-151); all in dtype qd.
int kas_contiguous_prefill(void* q, void* k, void* v, void* out, int B, int S, int Hq, int Hkv, int D, int qd,
                           void* stream)
{
    kernels::set_default_stream(static_cast<hipStream_t>(stream));
    const DType qt = static_cast<DType>(qd);
    Tensor      tq = Tensor::from_external(q, {B, S, Hq, D}, qt, Device::GPU);
    Tensor      tk = Tensor::from_external(k, {B, S, Hkv, D}, qt, Device::GPU);
    Tensor      tv = Tensor::from_external(v, {B, S, Hkv, D}, qt, Device::GPU);
    Tensor      to = Tensor::from_external(out, {B, S, Hq * D}, qt, Device::GPU);
    kernels::attention(tq, tk, tv, to, nullptr, Hkv, S, 0, nullptr);
    if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
    return 0;
}

// Chunked prefill through the paged branch: q [B,S,Hq,D] with a block table, after kernels::append_kv_cache.
int kas_paged_prefill(void* q, void* k_new, void* v_new, void* k_cache, void* v_cache, void* out,
                      const int* block_table, const int* context_lens, int B, int S, int Hq, int Hkv, int D, int N,
                      int max_blocks, int qd, int cd, void* stream)
{
    kernels::set_default_stream(static_cast<hipStream_t>(stream));
    const DType qt = static_cast<DType>(qd), ct = static_cast<DType>(cd);
    Tensor      tq = Tensor::from_external(q, {B, S, Hq, D}, qt, Device::GPU);
    Tensor      tk = Tensor::from_external(k_new, {B, S, Hkv, D}, qt, Device::GPU);
    Tensor      tv = Tensor::from_external(v_new, {B, S, Hkv, D}, qt, Device::GPU);
    Tensor      kc = Tensor::from_external(k_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    Tensor      vc = Tensor::from_external(v_cache, {N, 16, Hkv, D}, ct, Device::GPU);
    Tensor      to = Tensor::from_external(out, {B, S, Hq * D}, qt, Device::GPU);
    kernels::append_kv_cache(tk, tv, kc, vc, block_table, context_lens, max_blocks);
    if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
    kernels::attention(tq, kc, vc, to, const_cast<int*>(block_table), Hkv, S, max_blocks, context_lens);
    if (!kernels::last_error().empty()) return g_err = kernels::last_error(), -1;
    return 0;
}

}  // extern "C"
