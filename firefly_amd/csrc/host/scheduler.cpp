// scheduler.cpp - block allocator and continuous-batching scheduler (the producers of KV block tables).
//
// The block ids and context lengths it produces follow the reference (src/scheduler.cc):
//   BlockAllocator   LIFO free list seeded 0..N-1 (:13-21), eviction from the prefix cache on shortage (:26-36),
//                    blocks handed out from the back of the list (:38-42), freed blocks pushed back (:46-52)
//   add_request      prefix match -> block_table / context_len / radix_nodes (:66-74)
//   step             running requests gain the blocks their next step writes (:88-112 under
//                    PrefillBlocks::OnePerStep); pending requests, longest cached prefix first (stable sort), are
//                    admitted while a batch slot and the blocks of their first chunk are free (:114-160), a fully
//                    cached prompt giving back its last matched node so at least one token is computed (:124-133)
//   finish_request   release prefix references, insert prompt + generated tokens with the block table (:165-186)
// Under the default PrefillBlocks::PerChunk a request part-way through its prompt gains all the blocks of its next
// chunk before it runs; the reference gives it one block per step, which leaves later chunks of a long prompt
// without blocks for their tokens.
#include <algorithm>
#include <iostream>

#include "firefly/scheduler.h"

namespace firefly
{

BlockAllocator::BlockAllocator() = default;

void BlockAllocator::init(int total_blocks, RadixTree* tree)
{
    total_blocks_ = total_blocks;
    tree_ = tree;
    free_list_.resize(total_blocks > 0 ? static_cast<size_t>(total_blocks) : 0);
    for (int i = 0; i < total_blocks; ++i) free_list_[static_cast<size_t>(i)] = i;
}

void BlockAllocator::set_radix_tree(RadixTree* tree) { tree_ = tree; }

bool BlockAllocator::allocate(int num_blocks, std::vector<int>& out_blocks)
{
    if (num_blocks < 0) return false;
    const size_t want = static_cast<size_t>(num_blocks);
    if (free_list_.size() < want && tree_ != nullptr) tree_->evict(num_blocks - static_cast<int>(free_list_.size()));
    if (free_list_.size() < want) return false;
    for (size_t i = 0; i < want; ++i)
    {
        out_blocks.push_back(free_list_.back());
        free_list_.pop_back();
    }
    return true;
}

void BlockAllocator::free(const std::vector<int>& blocks)
{
    free_list_.insert(free_list_.end(), blocks.begin(), blocks.end());
}

int BlockAllocator::get_free_blocks() const { return static_cast<int>(free_list_.size()); }

Scheduler::Scheduler() = default;

void Scheduler::init(int max_context_blocks, int max_batch_size_limit, int max_prefill_chunk_size)
{
    init(max_context_blocks, max_batch_size_limit, max_prefill_chunk_size, PrefillBlocks::PerChunk);
}

void Scheduler::init(int max_context_blocks, int max_batch_size_limit, int max_prefill_chunk_size,
                     PrefillBlocks prefill_blocks)
{
    std::lock_guard<std::mutex> lock(mutex_);
    max_batch_ = max_batch_size_limit;
    max_chunk_ = max_prefill_chunk_size;
    prefill_blocks_ = prefill_blocks;
    tree_ = std::make_unique<RadixTree>(&allocator_);
    allocator_.init(max_context_blocks, tree_.get());
}

void Scheduler::add_request(RequestPtr req)
{
    std::lock_guard<std::mutex> lock(mutex_);
    RadixTree::MatchResult      m = tree_->match_prefix(req->prompt_tokens);
    req->block_table = std::move(m.matched_blocks);
    req->context_len = m.matched_tokens;
    req->radix_nodes = std::move(m.matched_nodes);
    pending_.push_back(std::move(req));
}

bool Scheduler::has_unfinished_requests()
{
    std::lock_guard<std::mutex> lock(mutex_);
    return !pending_.empty() || !active_.empty();
}

int Scheduler::free_blocks()
{
    std::lock_guard<std::mutex> lock(mutex_);
    return allocator_.get_free_blocks();
}

// KV positions the request's next step leaves in the cache: the next prefill chunk's end, or, once decoding, its
// whole sequence (the step appends the newest token at context_len = total - 1).
int Scheduler::step_tokens(const GenerationRequest& r) const
{
    if (!r.generated_tokens.empty()) return r.get_total_len();
    const int left = static_cast<int>(r.prompt_tokens.size()) - r.context_len;
    return r.context_len + std::min(left, max_chunk_);
}

// Blocks a running request must gain before its next step.  Decoding requests (and, under OnePerStep, prefilling
// ones too) gain one block when their sequence has reached the end of the blocks they hold; under PerChunk a
// prefilling request gains every block its next chunk writes.
int Scheduler::blocks_to_run(const GenerationRequest& r) const
{
    const int have = static_cast<int>(r.block_table.size());
    if (prefill_blocks_ == PrefillBlocks::PerChunk && r.generated_tokens.empty())
        return std::max(0, (step_tokens(r) + block_size_ - 1) / block_size_ - have);
    return r.get_total_len() >= have * block_size_ ? 1 : 0;
}

// Blocks a request part-way through its prompt still needs to hold the whole prompt (0 once decoding).
int Scheduler::prompt_blocks_left(const GenerationRequest& r) const
{
    if (!r.generated_tokens.empty()) return 0;
    const int want = (static_cast<int>(r.prompt_tokens.size()) + block_size_ - 1) / block_size_;
    return std::max(0, want - static_cast<int>(r.block_table.size()));
}

// Appends `blocks` new blocks to r's table (evicting from the prefix cache if the allocator must); false, and no
// change, if they cannot be had.
bool Scheduler::reserve(GenerationRequest& r, int blocks)
{
    if (blocks <= 0) return true;
    return allocator_.allocate(blocks, r.block_table);
}

// A prompt found whole in the prefix cache still needs one forward pass for its logits: give back the last
// matched node so that its tokens are computed again.
void Scheduler::uncache_last_node(GenerationRequest& r)
{
    const std::shared_ptr<TreeNode> node = r.radix_nodes.back();
    r.radix_nodes.pop_back();
    r.context_len -= static_cast<int>(node->tokens.size());
    r.block_table.resize(r.block_table.size() - node->block_indices.size());
    node->ref_count--;
}

// Admission of a pending request: a free batch slot and the blocks of its first chunk, both available now.
// Under PerChunk the whole prompt must fit beside what the admitted prompts still need (reserved_), counting
// blocks the prefix cache can give back; the reference (OnePerStep) counts free blocks against the first chunk
// only, so two long prompts admitted together can each wait forever for the blocks of their next chunk.
bool Scheduler::admit(GenerationRequest& r)
{
    if (r.context_len == static_cast<int>(r.prompt_tokens.size()) && !r.radix_nodes.empty()) uncache_last_node(r);
    const int need = (step_tokens(r) + block_size_ - 1) / block_size_ - static_cast<int>(r.block_table.size());
    if (static_cast<int>(active_.size()) >= max_batch_) return false;
    if (prefill_blocks_ == PrefillBlocks::PerChunk)
    {
        const int whole = prompt_blocks_left(r);
        if (whole + reserved_ > allocator_.get_free_blocks() + tree_->evictable_blocks()) return false;
        if (!reserve(r, need)) return false;
        reserved_ += whole - need;
    }
    else
    {
        if (need > allocator_.get_free_blocks()) return false;
        if (!reserve(r, need)) return false;
    }
    r.status = RequestStatus::ACTIVE;
    return true;
}

SchedulerBatch Scheduler::step()
{
    std::lock_guard<std::mutex> lock(mutex_);
    SchedulerBatch              batch;

    // Running requests first, in arrival order; one whose blocks cannot be had sits this step out.
    for (const RequestPtr& r : active_)
    {
        if (reserve(*r, blocks_to_run(*r)))
            batch.requests.push_back(r);
        else
            std::cerr << "firefly::Scheduler: request " << r->id << " waits for a free KV block this step" << std::endl;
    }

    // Then waiting requests, longest cached prefix first (a stable order among equals), until one does not fit.
    reserved_ = 0;
    for (const RequestPtr& r : active_) reserved_ += prompt_blocks_left(*r);
    pending_.sort([](const RequestPtr& x, const RequestPtr& y) { return x->context_len > y->context_len; });
    while (!pending_.empty() && admit(*pending_.front()))
    {
        batch.requests.push_back(pending_.front());
        active_.splice(active_.end(), pending_, pending_.begin());
    }
    return batch;
}

void Scheduler::finish_request(RequestPtr req)
{
    std::lock_guard<std::mutex> lock(mutex_);
    active_.remove(req);
    req->status = RequestStatus::FINISHED;
    // hand the whole sequence and its blocks to the prefix cache, which owns the blocks from now on
    tree_->decrement_ref_counts(req->radix_nodes);
    req->radix_nodes.clear();
    std::vector<int> sequence;
    sequence.reserve(req->prompt_tokens.size() + req->generated_tokens.size());
    sequence.insert(sequence.end(), req->prompt_tokens.begin(), req->prompt_tokens.end());
    sequence.insert(sequence.end(), req->generated_tokens.begin(), req->generated_tokens.end());
    tree_->insert(sequence, req->block_table);
    req->block_table.clear();
}

}  // namespace firefly
