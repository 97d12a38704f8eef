// engine_calls.cpp - the reference engine's uses of hal::Graph and hal::Result, compiled against this repository's
// headers (tests/test_hal.py builds and runs it on the CPU).
//
// decode_graph_setup() has the call shapes of the engine's decode-graph capture (src/engine.cc:137-166): capture
// with a lambda, test the result as a bool, print result.error().description(), warm the graph with
// `[[maybe_unused]] auto _ = graph.launch(stream)`, move the graph into a map.  decode_graph_launch() has those of
// the replay (src/engine.cc:329-333).  main() also checks Result<T>, Status and FIREFLY_TRY.  Without a GPU the
// capture fails inside the HIP runtime, which exercises the error path end to end.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <iostream>
#include <map>
#include <string>

#include "firefly/hal/error.h"
#include "firefly/hal/graph.h"
#include "firefly/kernels.h"

namespace
{

struct GraphData
{
    firefly::hal::Graph graph;
};

std::map<int, GraphData> graphs;

int decode_graph_setup(hipStream_t capture_stream, int bs, std::string& why)
{
    GraphData gd;
    firefly::kernels::set_default_stream(capture_stream);
    auto result = gd.graph.capture(capture_stream,
                                   [&]()
                                   {
                                       // the engine runs model_->forward(...) and kernels::argmax(...) here
                                   });
    firefly::kernels::set_default_stream(nullptr);
    if (!result)
    {
        std::cerr << "Failed to capture graph for batch size " << bs << ": " << result.error().description()
                  << std::endl;
        why = result.error().description();
        return 1;
    }
    [[maybe_unused]] auto _ = gd.graph.launch(capture_stream);
    (void)hipStreamSynchronize(capture_stream);
    graphs[bs] = std::move(gd);
    return 0;
}

int decode_graph_launch(const GraphData& gd, hipStream_t decode_stream, std::string& why)
{
    auto result = gd.graph.launch(decode_stream);
    if (!result)
    {
        std::cerr << "Graph Launch failed: " << result.error().description() << std::endl;
        why = result.error().description();
        return 1;
    }
    return 0;
}

firefly::hal::Result<int> half_of(int x)
{
    if (x % 2 != 0) return firefly::hal::unexpected(firefly::hal::Error{22, firefly::hal::ErrorCategory::Runtime, "odd"});
    return x / 2;
}

firefly::hal::Result<int> quarter_of(int x)
{
    const int h = FIREFLY_TRY(half_of(x));
    return FIREFLY_TRY(half_of(h));
}

firefly::hal::Status hip_status(hipError_t e) { return firefly::hal::check_hip(e); }

int failures = 0;

void expect(bool ok, const char* what)
{
    if (!ok)
    {
        std::printf("FAIL %s\n", what);
        ++failures;
    }
}

}  // namespace

int main()
{
    // Result<T> / Status / FIREFLY_TRY
    expect(quarter_of(8).has_value() && quarter_of(8).value() == 2, "quarter_of(8) == 2");
    auto q = quarter_of(6);  // 6 / 2 = 3 is odd: the second step fails and its error propagates
    expect(!q && q.error().code == 22 && std::strcmp(q.error().description(), "odd") == 0, "error propagates");
    expect(std::strcmp(q.error().name(), "RuntimeError") == 0, "runtime error name");
    expect(quarter_of(6).value_or(-1) == -1, "value_or");
    expect(static_cast<bool>(hip_status(hipSuccess)), "check_hip(hipSuccess) is ok");
    auto st = hip_status(hipErrorInvalidValue);
    expect(!st && st.error().category == firefly::hal::ErrorCategory::CUDA, "check_hip error category");
    expect(std::strcmp(st.error().description(), hipGetErrorString(hipErrorInvalidValue)) == 0,
           "HIP error described by the runtime");
    expect(st.error().location.line() > 0, "error records its location");
    firefly::hal::Result<std::string> moved = std::string("abc");
    firefly::hal::Result<std::string> copy = moved;
    expect(copy.value() == "abc" && moved.value() == "abc", "copy of a Result<std::string>");

    // hal::Graph with the engine's call shapes
    firefly::hal::Graph empty_graph;
    expect(empty_graph.empty(), "a new graph is empty");
    std::string why;
    expect(decode_graph_launch(GraphData{}, nullptr, why) == 1 && !why.empty(), "launching an empty graph fails");
    int  devices = 0;
    const bool gpu = hipGetDeviceCount(&devices) == hipSuccess && devices > 0;
    hipStream_t stream = nullptr;
    if (gpu) (void)hipStreamCreate(&stream);
    why.clear();
    const int rc = decode_graph_setup(stream, 8, why);
    if (gpu)
    {
        expect(rc == 0 && graphs.count(8) == 1 && !graphs[8].graph.empty(), "capture on a GPU");
        expect(decode_graph_launch(graphs[8], stream, why) == 0, "replay on a GPU");
        (void)hipStreamSynchronize(stream);
        (void)hipStreamDestroy(stream);
    }
    else
    {
        expect(rc == 1 && !why.empty(), "capture without a GPU reports a described error");
    }
    std::printf("%s (%s)\n", failures == 0 ? "OK" : "FAILED", gpu ? "gpu" : "no gpu");
    return failures == 0 ? 0 : 1;
}
