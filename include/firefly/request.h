// request.h - per-request state the scheduler keeps (reference include/firefly/request.h:11-43).
//
// Same fields and meaning: block_table holds the request's physical KV block ids in logical order (shared
// prefix blocks first), context_len the number of tokens already in the KV cache, radix_nodes the prefix-cache
// nodes the request holds a reference on.
#pragma once

#include <chrono>
#include <memory>
#include <string>
#include <vector>

namespace firefly
{

struct TreeNode;

enum class RequestStatus
{
    PENDING,
    ACTIVE,
    FINISHED
};

struct GenerationRequest
{
    std::string      id;
    std::vector<int> prompt_tokens;
    std::vector<int> generated_tokens;
    int              max_tokens;
    RequestStatus    status = RequestStatus::PENDING;
    std::string      utf8_buffer;

    std::vector<int>                       block_table;
    int                                    context_len = 0;
    std::vector<std::shared_ptr<TreeNode>> radix_nodes;

    std::chrono::steady_clock::time_point arrival_time;

    GenerationRequest(const std::string& request_id, const std::vector<int>& tokens, int max_tok)
        : id(request_id), prompt_tokens(tokens), max_tokens(max_tok), arrival_time(std::chrono::steady_clock::now())
    {
    }

    int get_total_len() const { return static_cast<int>(prompt_tokens.size() + generated_tokens.size()); }
};

using RequestPtr = std::shared_ptr<GenerationRequest>;

}  // namespace firefly
