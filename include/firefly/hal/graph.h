// graph.h - HIP graph capture of a decode step (reference include/firefly/hal/graph.h:17-158).
//
// Same interface as the reference's hal::Graph: capture(stream, fn) records everything fn launches on `stream`
// (thread-local capture mode, as the reference uses at :59) and instantiates it; launch(stream) replays it; both
// return Status (Result<void>) whose error() describes a failure; empty() is true while nothing is captured.  An
// exception thrown by fn ends the capture and is returned as a Runtime error.
//
// The path's kernels are capture-safe: no host synchronization, no allocation when a decode workspace is given,
// and no memset nodes (graph replays of memset nodes are avoided on purpose).
#pragma once

#include <hip/hip_runtime_api.h>

#include <functional>

#include "firefly/hal/error.h"
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

    Status capture(hipStream_t stream, std::function<void()> func);
    Status launch(hipStream_t stream) const;
    [[nodiscard]] bool empty() const { return exec_ == nullptr; }

private:
    void destroy();

    hipGraph_t     graph_ = nullptr;
    hipGraphExec_t exec_ = nullptr;
};

}  // namespace firefly::hal
