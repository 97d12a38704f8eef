// radix_tree.cpp - prefix cache of token sequences over 16-token KV blocks.
//
// Behaviour follows the reference's RadixTree (src/radix_tree.cc) step for step where it decides which physical
// blocks a request gets, because those ids end up in the block tables the KV kernels read:
//   match_prefix  (:13-95)   walk edges, keep only whole 16-token blocks of a partial edge match (splitting the
//                            edge there), take a reference and stamp the access time on every matched node
//   insert        (:111-181) walk edges, split at the first mismatching token (the split keeps ceil(len/16)
//                            blocks above), hang the unmatched suffix and the remaining blocks below
//   evict         (:202-235) repeatedly drop the least-recently-used unreferenced leaf (ties resolved by
//                            sorting the depth-first leaf list, as the reference does) and return its blocks
// One guard is added: a split never slices past the end of a node's block list (the reference would read out
// of bounds there).
#include <algorithm>
#include <iostream>

#include "firefly/radix_tree.h"
#include "firefly/scheduler.h"

namespace firefly
{

namespace
{

constexpr int kBlockTokens = 16;

size_t common_prefix(const std::vector<int>& edge, const std::vector<int>& seq, size_t from)
{
    const size_t limit = std::min(edge.size(), seq.size() - from);
    size_t       n = 0;
    while (n < limit && edge[n] == seq[from + n]) ++n;
    return n;
}

// Cut `node` after `keep_tokens` tokens, moving everything after the first `keep_blocks` blocks into a new child
// that inherits the children, reference count and access time.
void split_node(TreeNode& node, size_t keep_tokens, size_t keep_blocks)
{
    auto tail = std::make_shared<TreeNode>();
    tail->tokens.assign(node.tokens.begin() + static_cast<std::ptrdiff_t>(keep_tokens), node.tokens.end());
    if (keep_blocks < node.block_indices.size())
    {
        tail->block_indices.assign(node.block_indices.begin() + static_cast<std::ptrdiff_t>(keep_blocks),
                                   node.block_indices.end());
        node.block_indices.resize(keep_blocks);
    }
    tail->children = std::move(node.children);
    tail->ref_count.store(node.ref_count.load());
    tail->last_access_time = node.last_access_time;
    node.tokens.resize(keep_tokens);
    node.children.clear();
    node.children[tail->tokens.front()] = tail;
}

}  // namespace

RadixTree::RadixTree(BlockAllocator* allocator) : root_(std::make_shared<TreeNode>()), allocator_(allocator) {}

RadixTree::MatchResult RadixTree::match_prefix(const std::vector<int>& tokens)
{
    std::lock_guard<std::mutex> lock(mutex_);
    ++clock_;
    ++lookups_;
    MatchResult result;
    auto        node = root_;
    size_t      pos = 0;
    while (pos < tokens.size())
    {
        auto it = node->children.find(tokens[pos]);
        if (it == node->children.end()) break;
        auto         child = it->second;
        const size_t same = common_prefix(child->tokens, tokens, pos);
        const size_t whole = same / kBlockTokens * kBlockTokens;  // only whole blocks can be shared
        if (whole == 0) break;
        const bool partial = whole < child->tokens.size();
        if (partial) split_node(*child, whole, whole / kBlockTokens);
        child->ref_count++;
        child->last_access_time = clock_;
        result.matched_nodes.push_back(child);
        result.matched_blocks.insert(result.matched_blocks.end(), child->block_indices.begin(),
                                     child->block_indices.end());
        result.matched_tokens += static_cast<int>(child->tokens.size());
        if (partial) break;
        pos += same;
        node = child;
    }
    hits_tokens_ += static_cast<uint64_t>(result.matched_tokens);
    return result;
}

void RadixTree::decrement_ref_counts(const std::vector<std::shared_ptr<TreeNode>>& nodes)
{
    std::lock_guard<std::mutex> lock(mutex_);
    ++clock_;
    for (const auto& n : nodes)
    {
        if (n->ref_count > 0)
        {
            n->ref_count--;
            n->last_access_time = clock_;
        }
    }
}

void RadixTree::insert(const std::vector<int>& tokens, const std::vector<int>& blocks)
{
    std::lock_guard<std::mutex> lock(mutex_);
    ++clock_;
    auto   node = root_;
    size_t pos = 0;
    size_t block_pos = 0;
    while (pos < tokens.size())
    {
        auto it = node->children.find(tokens[pos]);
        if (it == node->children.end()) break;
        auto         child = it->second;
        const size_t same = common_prefix(child->tokens, tokens, pos);
        const size_t blocks_above = (same + kBlockTokens - 1) / kBlockTokens;
        if (same < child->tokens.size()) split_node(*child, same, blocks_above);
        pos += same;
        block_pos += blocks_above;
        node = child;
    }
    if (pos < tokens.size())
    {
        auto leaf = std::make_shared<TreeNode>();
        leaf->tokens.assign(tokens.begin() + static_cast<std::ptrdiff_t>(pos), tokens.end());
        if (block_pos < blocks.size())
            leaf->block_indices.assign(blocks.begin() + static_cast<std::ptrdiff_t>(block_pos), blocks.end());
        leaf->last_access_time = clock_;
        node->children[leaf->tokens.front()] = leaf;
    }
}

void RadixTree::find_evictable(const std::shared_ptr<TreeNode>& node, const std::shared_ptr<TreeNode>& parent,
                               std::vector<LeafRef>& out) const
{
    if (node != root_ && node->children.empty())
    {
        if (node->ref_count == 0) out.emplace_back(node, parent);
        return;
    }
    for (const auto& kv : node->children) find_evictable(kv.second, node, out);
}

int RadixTree::evict(int num_blocks_needed)
{
    std::lock_guard<std::mutex> lock(mutex_);
    int                         freed = 0;
    while (freed < num_blocks_needed)
    {
        std::vector<LeafRef> leaves;
        find_evictable(root_, nullptr, leaves);
        if (leaves.empty()) break;
        std::sort(leaves.begin(), leaves.end(),
                  [](const LeafRef& x, const LeafRef& y) { return x.first->last_access_time < y.first->last_access_time; });
        const LeafRef victim = leaves.front();
        freed += static_cast<int>(victim.first->block_indices.size());
        allocator_->free(victim.first->block_indices);
        if (victim.second) victim.second->children.erase(victim.first->tokens.front());
    }
    evicted_blocks_ += static_cast<uint64_t>(freed);
    return freed;
}

std::pair<int, bool> RadixTree::count_evictable(const TreeNode& node) const
{
    int  blocks = 0;
    bool whole = node.ref_count == 0;
    for (const auto& kv : node.children)
    {
        const auto [b, w] = count_evictable(*kv.second);
        blocks += b;
        whole = whole && w;
    }
    // evict() removes unreferenced leaves until none is left: a node goes once its whole subtree is unreferenced
    if (whole && &node != root_.get()) blocks += static_cast<int>(node.block_indices.size());
    return {blocks, whole};
}

int RadixTree::evictable_blocks() const
{
    std::lock_guard<std::mutex> lock(mutex_);
    return count_evictable(*root_).first;
}

void RadixTree::print_stats() const
{
    std::lock_guard<std::mutex> lock(mutex_);
    std::cout << "[RadixTree] lookups " << lookups_ << ", matched tokens " << hits_tokens_ << ", evicted blocks "
              << evicted_blocks_ << "\n";
}

}  // namespace firefly
