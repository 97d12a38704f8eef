// scheduler.cpp - block allocator and continuous-batching scheduler (the producers of KV block tables).
//
// Behaviour follows the reference (src/scheduler.cc) where it determines block ids and context lengths:
//   BlockAllocator   LIFO free list seeded 0..N-1 (:13-21), eviction from the prefix cache on shortage (:26-36),
//                    blocks handed out from the back of the list (:38-42), freed blocks pushed back (:46-52)
//   add_request      prefix match -> block_table / context_len / radix_nodes (:66-74)
//   step             active requests get one more block when their tokens fill the last (:88-112); pending
//                    requests, longest cached prefix first (stable sort), are admitted while a slot and the blocks
//                    for their next prefill chunk are available (:114-160), a fully cached prompt giving back its
//                    last matched node so at least one token is computed (:124-133)
//   finish_request   release prefix references, insert prompt + generated tokens with the block table (:165-186)
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
    std::lock_guard<std::mutex> lock(mutex_);
    max_batch_ = max_batch_size_limit;
    max_chunk_ = max_prefill_chunk_size;
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

SchedulerBatch Scheduler::step()
{
    std::lock_guard<std::mutex> lock(mutex_);
    SchedulerBatch              batch;

    // running requests: a new block once the tokens so far fill every block they have
    for (const RequestPtr& req : active_)
    {
        const size_t have = req->block_table.size();
        if (static_cast<size_t>(req->get_total_len()) < have * static_cast<size_t>(block_size_))
        {
            batch.requests.push_back(req);
            continue;
        }
        std::vector<int> one;
        if (allocator_.allocate(1, one))
        {
            req->block_table.push_back(one.front());
            batch.requests.push_back(req);
        }
        else
        {
            std::cerr << "[Warning] Out of memory during continuous batching decode!" << std::endl;
        }
    }

    // waiting requests, longest cached prefix first
    pending_.sort([](const RequestPtr& x, const RequestPtr& y) { return x->context_len > y->context_len; });
    for (auto it = pending_.begin(); it != pending_.end();)
    {
        const RequestPtr req = *it;
        int unmatched = static_cast<int>(req->prompt_tokens.size()) - req->context_len;
        if (unmatched == 0 && !req->radix_nodes.empty())
        {
            // fully cached prompt: recompute its last node so the model produces logits
            const std::shared_ptr<TreeNode> last = req->radix_nodes.back();
            req->context_len -= static_cast<int>(last->tokens.size());
            req->block_table.resize(req->block_table.size() - last->block_indices.size());
            last->ref_count--;
            req->radix_nodes.pop_back();
            unmatched = static_cast<int>(req->prompt_tokens.size()) - req->context_len;
        }
        const int chunk = std::min(unmatched, max_chunk_);
        const int target = req->context_len + chunk;
        const int needed = (target + block_size_ - 1) / block_size_ - static_cast<int>(req->block_table.size());
        if (static_cast<int>(active_.size()) < max_batch_ && needed <= allocator_.get_free_blocks())
        {
            std::vector<int> got;
            if (needed == 0 || allocator_.allocate(needed, got))
            {
                req->block_table.insert(req->block_table.end(), got.begin(), got.end());
                req->status = RequestStatus::ACTIVE;
                active_.push_back(req);
                batch.requests.push_back(req);
                it = pending_.erase(it);
                continue;
            }
        }
        break;  // no room for this request's next chunk: stop admitting
    }
    return batch;
}

void Scheduler::finish_request(RequestPtr req)
{
    std::lock_guard<std::mutex> lock(mutex_);
    req->status = RequestStatus::FINISHED;
    tree_->decrement_ref_counts(req->radix_nodes);
    req->radix_nodes.clear();
    std::vector<int> all = req->prompt_tokens;
    all.insert(all.end(), req->generated_tokens.begin(), req->generated_tokens.end());
    tree_->insert(all, req->block_table);
    req->block_table.clear();  // the prefix cache owns the blocks from now on
    auto it = std::find(active_.begin(), active_.end(), req);
    if (it != active_.end()) active_.erase(it);
}

}  // namespace firefly
