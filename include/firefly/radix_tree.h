// radix_tree.h - prefix cache over token sequences whose edges own whole 16-token KV blocks.
//
// Same interface and observable behaviour as the reference RadixTree (include/firefly/radix_tree.h:14-109,
// src/radix_tree.cc): match_prefix() shares only whole 16-token blocks (a partial match is cut back to a block
// boundary, splitting the node there) and takes a reference on every matched node; insert() adds a finished
// sequence, splitting nodes where it diverges; evict() frees the blocks of least-recently-used unreferenced leaves
// back to the BlockAllocator.  The block ids a match returns are what every sharing request's block table starts
// with, which is how prefix pages are shared between sequences in the paged KV cache.
#pragma once

#include <atomic>
#include <cstdint>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <utility>
#include <vector>

#include "firefly/types.h"

namespace firefly
{

class BlockAllocator;

struct TreeNode
{
    std::vector<int> tokens;         // edge label
    std::vector<int> block_indices;  // physical blocks holding those tokens' K/V
    std::atomic<int> ref_count{0};   // requests currently using this node
    uint64_t         last_access_time{0};

    std::unordered_map<int, std::shared_ptr<TreeNode>> children;  // keyed by the child's first token

    TreeNode() = default;
};

class FIREFLY_API RadixTree
{
public:
    explicit RadixTree(BlockAllocator* allocator);

    struct MatchResult
    {
        std::vector<std::shared_ptr<TreeNode>> matched_nodes;
        std::vector<int>                       matched_blocks;
        int                                    matched_tokens = 0;
    };

    // Longest block-aligned prefix of `tokens` in the tree; increments the matched nodes' ref_count.
    MatchResult match_prefix(const std::vector<int>& tokens);

    // Add a sequence and the blocks holding it (blocks[i] holds tokens [16i, 16i + 16)).
    void insert(const std::vector<int>& tokens, const std::vector<int>& blocks);

    // Release references taken by match_prefix.
    void decrement_ref_counts(const std::vector<std::shared_ptr<TreeNode>>& nodes);

    // Evict least-recently-used unreferenced leaves until num_blocks_needed blocks are freed (or nothing is
    // evictable); returns the number of blocks freed.
    int evict(int num_blocks_needed);

    // Blocks evict() could free now: those of every node whose subtree holds no referenced node.  Not in the
    // reference; the scheduler's PrefillBlocks::PerChunk admission counts them.
    int evictable_blocks() const;

    void print_stats() const;

private:
    using LeafRef = std::pair<std::shared_ptr<TreeNode>, std::shared_ptr<TreeNode>>;  // (leaf, parent)

    void find_evictable(const std::shared_ptr<TreeNode>& node, const std::shared_ptr<TreeNode>& parent,
                        std::vector<LeafRef>& out) const;
    // (blocks evictable within node's subtree, whether the whole subtree is unreferenced)
    std::pair<int, bool> count_evictable(const TreeNode& node) const;

    std::shared_ptr<TreeNode> root_;
    BlockAllocator*           allocator_;
    mutable std::mutex        mutex_;
    uint64_t                  clock_ = 0;
    uint64_t                  hits_tokens_ = 0, lookups_ = 0, evicted_blocks_ = 0;
};

}  // namespace firefly
