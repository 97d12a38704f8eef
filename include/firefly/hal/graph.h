// graph.h - HIP graph capture of a decode step (reference include/firefly/hal/graph.h:54-88).
//
// Same use as the reference's hal::Graph: capture(stream, fn) records everything fn launches on `stream`
// (thread-local capture mode, as the reference uses at :59), instantiates it, and launch(stream) replays it.  The
// reference returns Result<void>; here capture/launch return true on success and error() holds the message.
// The path's kernels are capture-safe: no host synchronization, no allocation when a decode workspace is given,
// and no memset nodes (graph replays of memset nodes are avoided on purpose).
#pragma once

#include <hip/hip_runtime_api.h>

#include <functional>
#include <string>

#include "firefly/types.h"

namespace firefly::hal
{

class FIREFLY_API Graph
{
public:
    Graph() = default;
    ~Graph();
    Graph(Graph&& other) noexcept;
    Graph& operator=(Graph&& other) noexcept;
    Graph(const Graph&) = delete;
    Graph& operator=(const Graph&) = delete;

    bool               capture(hipStream_t stream, const std::function<void()>& fn);
    bool               launch(hipStream_t stream) const;
    bool               captured() const { return exec_ != nullptr; }
    const std::string& error() const { return error_; }

private:
    void destroy();

    hipGraph_t          graph_ = nullptr;
    hipGraphExec_t      exec_ = nullptr;
    mutable std::string error_;
};

}  // namespace firefly::hal
