// decode_step_shim.cpp - C entry points over firefly::DecodeBatch and firefly::hal::Graph for
// tests/test_gpu_decode_step.py: the engine's decode step (src/engine.cc:279-351) with this library, i.e. pack the
// scheduled requests' context lengths and block tables, upload them, and replay one captured graph that runs, per
// layer, kernels::append_kv_cache then kernels::attention on the packed device buffers.
#include <memory>
#include <string>
#include <vector>

#include "firefly/decode_batch.h"
#include "firefly/hal/graph.h"
#include "firefly/kernels.h"

using namespace firefly;

namespace
{

struct Step
{
    std::unique_ptr<DecodeBatch> batch;
    hal::Graph                   graph;
    std::string                  err;
};

}  // namespace

extern "C" {

void* dss_create(int capacity, int stride)
{
    auto* s = new Step;
    s->batch = std::make_unique<DecodeBatch>(capacity, stride);
    if (!s->batch->ok())
    {
        delete s;
        return nullptr;
    }
    return s;
}

void dss_destroy(void* h) { delete static_cast<Step*>(h); }

const char* dss_error(void* h) { return static_cast<Step*>(h)->err.c_str(); }

// n requests: context_len[i], block-table lengths nblk[i], blocks concatenated in `blocks`.
int dss_pack(void* h, int n, const int* context_len, const int* nblk, const int* blocks)
{
    auto*                                      s = static_cast<Step*>(h);
    std::vector<std::unique_ptr<GenerationRequest>> reqs;
    std::vector<const GenerationRequest*>       ptrs;
    size_t                                      off = 0;
    for (int i = 0; i < n; ++i)
    {
        auto r = std::make_unique<GenerationRequest>("r" + std::to_string(i), std::vector<int>{}, 1);
        r->context_len = context_len[i];
        r->block_table.assign(blocks + off, blocks + off + nblk[i]);
        off += static_cast<size_t>(nblk[i]);
        ptrs.push_back(r.get());
        reqs.push_back(std::move(r));
    }
    return s->batch->pack(ptrs);
}

int dss_upload(void* h, void* stream) { return static_cast<Step*>(h)->batch->upload(static_cast<hipStream_t>(stream)) ? 0 : -1; }

long long dss_last_upload_bytes(void* h) { return static_cast<long long>(static_cast<Step*>(h)->batch->last_upload_bytes()); }

const int* dss_host_table(void* h) { return static_cast<Step*>(h)->batch->host_block_table(); }
const int* dss_host_ctx(void* h) { return static_cast<Step*>(h)->batch->host_context_lens(); }

// Per layer l: q[l] [cap,1,Hq,D], k_new[l]/v_new[l] [cap,1,Hkv,D], caches[l] [N,16,Hkv,D] (dtype dt), out[l]
// [cap,1,Hq*D].  eager = 1 runs the step on `stream`; 0 captures it into the step's graph.
int dss_step(void* h, int eager, int layers, void** q, void** k_new, void** v_new, void** kc, void** vc, void** out,
             int Hq, int Hkv, int D, int N, int dt, void* stream)
{
    auto*       s = static_cast<Step*>(h);
    const int   cap = s->batch->batch_capacity(), stride = s->batch->stride();
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto        body = [&]()
    {
        kernels::set_default_stream(st);
        for (int l = 0; l < layers; ++l)
        {
            const DType t = static_cast<DType>(dt);
            Tensor      tq = Tensor::from_external(q[l], {cap, 1, Hq, D}, t, Device::GPU);
            Tensor      tk = Tensor::from_external(k_new[l], {cap, 1, Hkv, D}, t, Device::GPU);
            Tensor      tv = Tensor::from_external(v_new[l], {cap, 1, Hkv, D}, t, Device::GPU);
            Tensor      kcache = Tensor::from_external(kc[l], {N, 16, Hkv, D}, t, Device::GPU);
            Tensor      vcache = Tensor::from_external(vc[l], {N, 16, Hkv, D}, t, Device::GPU);
            Tensor      to = Tensor::from_external(out[l], {cap, 1, Hq * D}, t, Device::GPU);
            kernels::append_kv_cache(tk, tv, kcache, vcache, s->batch->device_block_table(),
                                     s->batch->device_context_lens(), stride);
            kernels::attention(tq, kcache, vcache, to, const_cast<int32_t*>(s->batch->device_block_table()), Hkv, 1,
                               stride, s->batch->device_context_lens());
        }
    };
    if (eager)
    {
        body();
        if (!kernels::last_error().empty()) return s->err = kernels::last_error(), -1;
        return 0;
    }
    auto result = s->graph.capture(st, body);
    if (!result) return s->err = result.error().description(), -1;
    if (!kernels::last_error().empty()) return s->err = kernels::last_error(), -1;
    return 0;
}

int dss_launch(void* h, void* stream)
{
    auto* s = static_cast<Step*>(h);
    auto result = s->graph.launch(static_cast<hipStream_t>(stream));
    if (!result) return s->err = result.error().description(), -1;
    return 0;
}

}  // extern "C"
