// scheduler.h - KV block allocator and the continuous-batching scheduler that builds block tables.
//
// Same interfaces and behaviour as the reference (include/firefly/scheduler.h:13-74, src/scheduler.cc):
//   BlockAllocator  LIFO free list of physical block ids 0..N-1 (the first allocations return N-1, N-2, ...);
//                   on shortage it asks the radix tree to evict first.  Not internally locked (the scheduler
//                   holds its mutex around every use).
//   Scheduler       add_request() matches the prompt against the prefix cache (shared blocks, context_len);
//                   step() gives running requests the blocks their next step writes and admits pending requests
//                   (longest cached prefix first) with blocks for their first prefill chunk; finish_request()
//                   returns the sequence and its blocks to the prefix cache.  PrefillBlocks selects how later
//                   prefill chunks are sized (the reference under-sizes them).
#pragma once

#include <cstdint>
#include <list>
#include <memory>
#include <mutex>
#include <vector>

#include "firefly/radix_tree.h"
#include "firefly/request.h"

namespace firefly
{

class FIREFLY_API BlockAllocator
{
public:
    BlockAllocator();
    void init(int total_blocks, RadixTree* tree = nullptr);
    void set_radix_tree(RadixTree* tree);

    // Appends num_blocks ids to out_blocks; false (nothing appended) if they cannot be had even after eviction.
    bool allocate(int num_blocks, std::vector<int>& out_blocks);
    void free(const std::vector<int>& blocks);
    int  get_free_blocks() const;

private:
    std::vector<int> free_list_;  // back = next id handed out
    int              total_blocks_ = 0;
    RadixTree*       tree_ = nullptr;
};

struct SchedulerBatch
{
    std::vector<RequestPtr> requests;
};

// How a request that is part-way through its prompt gets the blocks of its next prefill chunk.
enum class PrefillBlocks : uint8_t
{
    // Before each chunk runs, the request holds a block for every position the chunk writes, and a prompt is
    // admitted only when the free and evictable blocks cover the rest of it on top of what the running prompts
    // still need, so prompts part-way through prefill never wait on each other for blocks.  Default.
    PerChunk,
    // The reference's rule (src/scheduler.cc:88-99,137-149): only the admitting chunk is sized; afterwards a
    // running request gains at most one block per step, so with chunk C a prompt longer than C + 16 tokens runs
    // later chunks past the end of its block table (their K/V are not stored and their keys are not attended).
    // Kept for block-id compatibility with the reference.
    OnePerStep,
};

class FIREFLY_API Scheduler
{
public:
    Scheduler();
    // max_context_blocks: pool size in blocks; max_batch_size_limit: cap on active requests;
    // max_prefill_chunk_size: tokens a request may prefill in one step.  The three-argument form is the
    // reference's (same symbol) and selects PrefillBlocks::PerChunk.
    void init(int max_context_blocks, int max_batch_size_limit, int max_prefill_chunk_size);
    void init(int max_context_blocks, int max_batch_size_limit, int max_prefill_chunk_size,
              PrefillBlocks prefill_blocks);

    void add_request(RequestPtr req);
    SchedulerBatch step();
    void finish_request(RequestPtr req);
    bool has_unfinished_requests();

    // Free blocks right now (diagnostics and tests).
    int free_blocks();

private:
    int  step_tokens(const GenerationRequest& r) const;
    int  blocks_to_run(const GenerationRequest& r) const;
    int  prompt_blocks_left(const GenerationRequest& r) const;
    bool reserve(GenerationRequest& r, int blocks);
    void uncache_last_node(GenerationRequest& r);
    bool admit(GenerationRequest& r);

    std::mutex            mutex_;
    std::list<RequestPtr> pending_;
    std::list<RequestPtr> active_;

    BlockAllocator             allocator_;
    std::unique_ptr<RadixTree> tree_;
    int                        block_size_ = 16;
    int                        max_batch_ = 64;
    int                        max_chunk_ = 256;
    PrefillBlocks              prefill_blocks_ = PrefillBlocks::PerChunk;
    int                        reserved_ = 0;  // PerChunk: blocks the admitted prompts still need (this step)
};

}  // namespace firefly
