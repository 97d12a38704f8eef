// sched_driver.cpp - C driver over the firefly block-table producers.  TEST INFRASTRUCTURE ONLY.
//
// The same source is compiled twice: against the reference's own scheduler and radix tree (its
// include/firefly/{scheduler,radix_tree,request}.h with src/scheduler.cc and src/radix_tree.cc, into
// oracle/_ref/libref_sched.so by `make -C oracle ref`) and against this repository's implementation (include/firefly
// with firefly_amd/libffkv.so, by tests/conftest.py).  Tests run identical scripted operations through both and
// compare every returned block id, context length and count.  Built over this repository (FFKV_SCHED_POLICY defined)
// it can also select the scheduler's PrefillBlocks policy.
//
// The engine emulation in sd_engine_step follows the reference engine loop's bookkeeping (src/engine.cc:219-351):
// a request without generated tokens prefills min(unmatched, chunk) tokens and produces its first token when the
// prompt is done; a request with generated tokens decodes one token; requests reaching max_tokens are finished.
// Generated token ids are a fixed function of (request id, position) so both builds see the same sequences.
#include <cstdint>
#include <map>
#include <memory>
#include <vector>

#include "firefly/radix_tree.h"
#include "firefly/request.h"
#include "firefly/scheduler.h"

using namespace firefly;

namespace
{

struct Serving
{
    Scheduler                    sched;
    std::map<int, RequestPtr>    reqs;
    int                          chunk = 256;
};

struct Pool
{
    BlockAllocator                                       alloc;
    std::unique_ptr<RadixTree>                           tree;
    std::map<int, std::vector<std::shared_ptr<TreeNode>>> matches;
    int                                                  next_match = 0;
};

int next_token(int id, size_t pos) { return static_cast<int>((static_cast<uint64_t>(id) * 7919u + pos * 104729u) % 50000u); }

// [n, then per request: id, context_len, generated count, n_blocks, blocks...]; returns ints written (or -needed).
int serialize(const std::vector<RequestPtr>& reqs, const std::map<int, RequestPtr>& by_id, int* out, int cap)
{
    std::vector<int> v;
    v.push_back(static_cast<int>(reqs.size()));
    for (const RequestPtr& r : reqs)
    {
        int id = -1;
        for (const auto& kv : by_id)
            if (kv.second == r) id = kv.first;
        v.push_back(id);
        v.push_back(r->context_len);
        v.push_back(static_cast<int>(r->generated_tokens.size()));
        v.push_back(static_cast<int>(r->block_table.size()));
        v.insert(v.end(), r->block_table.begin(), r->block_table.end());
    }
    if (static_cast<int>(v.size()) > cap) return -static_cast<int>(v.size());
    for (size_t i = 0; i < v.size(); ++i) out[i] = v[i];
    return static_cast<int>(v.size());
}

}  // namespace

extern "C" {

// ---- scheduler + emulated engine -------------------------------------------------------------------------

// per_chunk = 1 selects this repository's PrefillBlocks::PerChunk (later prefill chunks get all their blocks);
// 0 the reference's one-block-per-step rule, the only one the reference build has (it returns NULL for 1).
void* sd_create_policy(int total_blocks, int max_batch, int max_chunk, int per_chunk)
{
#ifndef FFKV_SCHED_POLICY
    if (per_chunk) return nullptr;
#endif
    auto* s = new Serving();
    s->chunk = max_chunk;
#ifdef FFKV_SCHED_POLICY
    s->sched.init(total_blocks, max_batch, max_chunk, per_chunk ? PrefillBlocks::PerChunk : PrefillBlocks::OnePerStep);
#else
    s->sched.init(total_blocks, max_batch, max_chunk);
#endif
    return s;
}

// The reference's rule, in both builds (block ids comparable with the reference).
void* sd_create(int total_blocks, int max_batch, int max_chunk) { return sd_create_policy(total_blocks, max_batch, max_chunk, 0); }

void sd_destroy(void* h) { delete static_cast<Serving*>(h); }

void sd_add(void* h, int id, const int* tokens, int n, int max_tokens)
{
    auto* s = static_cast<Serving*>(h);
    auto  r = std::make_shared<GenerationRequest>(std::to_string(id), std::vector<int>(tokens, tokens + n), max_tokens);
    s->reqs[id] = r;
    s->sched.add_request(r);
}

// Request state: [context_len, generated, n_blocks, blocks...]; returns ints written (or -needed, -1 if unknown).
int sd_request(void* h, int id, int* out, int cap)
{
    auto* s = static_cast<Serving*>(h);
    auto  it = s->reqs.find(id);
    if (it == s->reqs.end()) return -1;
    const RequestPtr& r = it->second;
    std::vector<int>  v{r->context_len, static_cast<int>(r->generated_tokens.size()),
                       static_cast<int>(r->block_table.size())};
    v.insert(v.end(), r->block_table.begin(), r->block_table.end());
    if (static_cast<int>(v.size()) > cap) return -static_cast<int>(v.size());
    for (size_t i = 0; i < v.size(); ++i) out[i] = v[i];
    return static_cast<int>(v.size());
}

// One engine iteration: schedule, serialize the batch as scheduled (block tables the kernels would read), then
// advance every request and finish those at max_tokens.  Returns ints written.
int sd_engine_step(void* h, int* out, int cap)
{
    auto*          s = static_cast<Serving*>(h);
    SchedulerBatch batch = s->sched.step();
    const int      written = serialize(batch.requests, s->reqs, out, cap);
    for (const RequestPtr& r : batch.requests)
    {
        int id = 0;
        for (const auto& kv : s->reqs)
            if (kv.second == r) id = kv.first;
        if (r->generated_tokens.empty())
        {
            const int unmatched = static_cast<int>(r->prompt_tokens.size()) - r->context_len;
            const int len = unmatched < s->chunk ? unmatched : s->chunk;
            r->context_len += len;
            if (r->context_len == static_cast<int>(r->prompt_tokens.size()))
                r->generated_tokens.push_back(next_token(id, r->prompt_tokens.size()));
        }
        else
        {
            r->generated_tokens.push_back(next_token(id, r->prompt_tokens.size() + r->generated_tokens.size()));
            r->context_len += 1;
        }
    }
    for (const RequestPtr& r : batch.requests)
        if (!r->generated_tokens.empty() && r->generated_tokens.size() >= static_cast<size_t>(r->max_tokens))
            s->sched.finish_request(r);
    return written;
}

int sd_unfinished(void* h) { return static_cast<Serving*>(h)->sched.has_unfinished_requests() ? 1 : 0; }

// ---- allocator + prefix cache directly -------------------------------------------------------------------

void* sd_pool_create(int total_blocks)
{
    auto* p = new Pool();
    p->tree = std::make_unique<RadixTree>(&p->alloc);
    p->alloc.init(total_blocks, p->tree.get());
    return p;
}

void sd_pool_destroy(void* h) { delete static_cast<Pool*>(h); }

// Appends n ids to out; returns 1 on success, 0 if the allocator refused.
int sd_alloc(void* h, int n, int* out)
{
    std::vector<int> got;
    if (!static_cast<Pool*>(h)->alloc.allocate(n, got)) return 0;
    for (size_t i = 0; i < got.size(); ++i) out[i] = got[i];
    return 1;
}

void sd_free(void* h, const int* blocks, int n) { static_cast<Pool*>(h)->alloc.free(std::vector<int>(blocks, blocks + n)); }

int sd_free_count(void* h) { return static_cast<Pool*>(h)->alloc.get_free_blocks(); }

// Match; writes matched blocks to out_blocks (up to cap) and the token count to *matched_tokens; returns a handle
// for sd_release (its node references are held until then) or -needed if cap is too small.
int sd_match(void* h, const int* tokens, int n, int* out_blocks, int cap, int* matched_tokens, int* n_blocks)
{
    auto* p = static_cast<Pool*>(h);
    auto  m = p->tree->match_prefix(std::vector<int>(tokens, tokens + n));
    if (static_cast<int>(m.matched_blocks.size()) > cap) return -static_cast<int>(m.matched_blocks.size());
    for (size_t i = 0; i < m.matched_blocks.size(); ++i) out_blocks[i] = m.matched_blocks[i];
    *matched_tokens = m.matched_tokens;
    *n_blocks = static_cast<int>(m.matched_blocks.size());
    const int id = p->next_match++;
    p->matches[id] = m.matched_nodes;
    return id;
}

void sd_release(void* h, int match_id)
{
    auto* p = static_cast<Pool*>(h);
    auto  it = p->matches.find(match_id);
    if (it == p->matches.end()) return;
    p->tree->decrement_ref_counts(it->second);
    p->matches.erase(it);
}

void sd_insert(void* h, const int* tokens, int n, const int* blocks, int nb)
{
    static_cast<Pool*>(h)->tree->insert(std::vector<int>(tokens, tokens + n), std::vector<int>(blocks, blocks + nb));
}

int sd_evict(void* h, int n) { return static_cast<Pool*>(h)->tree->evict(n); }

}  // extern "C"
