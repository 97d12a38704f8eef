// sched_sanitize.cpp - BlockAllocator / RadixTree / Scheduler under AddressSanitizer and UBSan
// (tests/test_sanitize.py builds it with g++ -fsanitize=address,undefined and runs it on the CPU).
//
// Seeded serving workloads (shared prompt prefixes, long prompts over small prefill chunks, pools small enough to
// force eviction) run through the scheduler with both PrefillBlocks policies and an engine emulation like the
// reference loop's bookkeeping (src/engine.cc:219-351), then random allocator / prefix-cache operations.  Besides
// the sanitizers' own checks, every step verifies: block ids in range, no id twice in one
// request's table, free blocks never above the pool size.  (A workload need not drain: admission compares a
// chunk's blocks with the free list without evicting cached blocks, as the reference does, so a pending request
// can wait forever once cached prefixes fill the pool.)
#include <algorithm>
#include <cstdio>
#include <map>
#include <memory>
#include <random>
#include <set>
#include <vector>

#include "firefly/radix_tree.h"
#include "firefly/request.h"
#include "firefly/scheduler.h"

using namespace firefly;

namespace
{

int failures = 0;

void check(bool ok, const char* what, int seed)
{
    if (!ok && failures++ < 20) std::printf("FAIL seed %d: %s\n", seed, what);
}

void serving(int seed, PrefillBlocks policy)
{
    std::mt19937 rng(seed);
    auto         uni = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
    const int    total = uni(120, 600), max_batch = uni(2, 10), chunk = 16 * uni(1, 16);
    Scheduler    sched;
    sched.init(total, max_batch, chunk, policy);
    std::vector<std::vector<int>> prefixes(3);
    for (auto& p : prefixes)
        for (int i = uni(16, 200); i > 0; --i) p.push_back(uni(1, 30000));
    std::map<RequestPtr, int> live;  // keeps every request alive until it finishes
    int                       next_id = 0, steps = 0;
    for (; steps < 5000; ++steps)
    {
        if (next_id < 40 && uni(0, 3) == 0)
        {
            std::vector<int> toks(prefixes[uni(0, 2)]);
            toks.resize(uni(1, static_cast<int>(toks.size())));
            for (int i = uni(1, 300); i > 0; --i) toks.push_back(uni(1, 30000));
            auto r = std::make_shared<GenerationRequest>(std::to_string(next_id), toks, uni(1, 12));
            live[r] = next_id++;
            sched.add_request(r);
        }
        SchedulerBatch batch = sched.step();
        check(sched.free_blocks() >= 0 && sched.free_blocks() <= total, "free blocks within the pool", seed);
        for (const RequestPtr& r : batch.requests)
        {
            std::set<int> own(r->block_table.begin(), r->block_table.end());
            check(own.size() == r->block_table.size(), "no block twice in one table", seed);
            for (int blk : r->block_table) check(blk >= 0 && blk < total, "block id in range", seed);
            // the engine's bookkeeping: a prefill chunk, or one decoded token
            if (r->generated_tokens.empty())
            {
                const int left = static_cast<int>(r->prompt_tokens.size()) - r->context_len;
                r->context_len += std::min(left, chunk);
                if (r->context_len == static_cast<int>(r->prompt_tokens.size())) r->generated_tokens.push_back(7);
            }
            else
            {
                r->generated_tokens.push_back(uni(1, 30000));
                r->context_len += 1;
            }
        }
        for (const RequestPtr& r : batch.requests)
            if (!r->generated_tokens.empty() && static_cast<int>(r->generated_tokens.size()) >= r->max_tokens)
            {
                sched.finish_request(r);
                live.erase(r);
            }
        if (next_id >= 40 && !sched.has_unfinished_requests()) break;
    }
}

void pool_ops(int seed)
{
    std::mt19937   rng(seed);
    auto           uni = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
    const int      total = 64;
    BlockAllocator alloc;
    RadixTree      tree(&alloc);
    alloc.init(total, &tree);
    std::vector<std::vector<std::shared_ptr<TreeNode>>> held;
    std::vector<std::vector<int>>                       base(5);
    for (auto& b : base)
        for (int i = uni(8, 90); i > 0; --i) b.push_back(uni(0, 3));
    int next_block = 0;
    for (int op = 0; op < 400; ++op)
    {
        std::vector<int> seq(base[uni(0, 4)]);
        seq.resize(uni(1, static_cast<int>(seq.size())));
        const int kind = uni(0, 9);
        if (kind < 3 && next_block < 1000)
        {
            std::vector<int> got;
            const int        nb = (static_cast<int>(seq.size()) + 15) / 16;
            if (alloc.allocate(nb, got)) tree.insert(seq, got);
            next_block += nb;
        }
        else if (kind < 6)
        {
            RadixTree::MatchResult m = tree.match_prefix(seq);
            check(m.matched_tokens % 16 == 0 && m.matched_blocks.size() * 16 == static_cast<size_t>(m.matched_tokens),
                  "block-aligned match", seed);
            held.push_back(m.matched_nodes);
        }
        else if (kind < 8 && !held.empty())
        {
            const size_t i = static_cast<size_t>(uni(0, static_cast<int>(held.size()) - 1));
            tree.decrement_ref_counts(held[i]);
            held.erase(held.begin() + static_cast<long>(i));
        }
        else
        {
            tree.evict(uni(1, 6));
        }
        check(alloc.get_free_blocks() <= total, "free blocks within the pool", seed);
    }
    for (auto& h : held) tree.decrement_ref_counts(h);
    tree.evict(total);
}

}  // namespace

int main()
{
    for (int seed = 0; seed < 24; ++seed)
    {
        serving(seed, PrefillBlocks::PerChunk);
        serving(seed, PrefillBlocks::OnePerStep);
        pool_ops(seed);
    }
    std::printf("%s\n", failures == 0 ? "OK" : "FAILED");
    return failures == 0 ? 0 : 1;
}
