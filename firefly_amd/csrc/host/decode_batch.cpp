// decode_batch.cpp - decode-step packing (DecodeBatch) and HIP graph capture (hal::Graph).
//
// Packing follows src/engine.cc:296-312 (slot i <- request i's context_len and block_table, other slots padded
// with context_len 0 and block -1); the upload copies only the rows' live width instead of the whole
// pool-stride table (src/engine.cc:317-322).  Graph follows include/firefly/hal/graph.h:54-120.
#include "firefly/decode_batch.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <utility>

#include "ffkv_internal.h"
#include "firefly/hal/graph.h"

namespace firefly
{

DecodeBatch::DecodeBatch(int batch_capacity, int max_context_blocks)
    : capacity_(batch_capacity > 0 ? batch_capacity : 0), stride_(max_context_blocks > 0 ? max_context_blocks : 0)
{
    if (capacity_ == 0 || stride_ == 0) return;
    lens_rows_ = (capacity_ + stride_ - 1) / stride_;
    const size_t lens = static_cast<size_t>(lens_rows_) * stride_;
    const size_t all = (lens + static_cast<size_t>(capacity_) * stride_) * sizeof(int32_t);
    if (hipHostMalloc(reinterpret_cast<void**>(&h_all_), all, hipHostMallocMapped) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&d_all_), all) != hipSuccess)
    {
        release();
        return;
    }
    // the staging's address on the device, which upload's copy kernel reads; without it upload copies by DMA
    if (hipHostGetDevicePointer(reinterpret_cast<void**>(&h_dev_), h_all_, 0) != hipSuccess) h_dev_ = nullptr;
    h_context_lens_ = h_all_;
    h_block_table_ = h_all_ + lens;
    d_context_lens_ = d_all_;
    d_block_table_ = d_all_ + lens;
    // A padded table everywhere before the first upload, and device buffers that hold it from the start.
    std::fill(h_all_, h_all_ + lens, 0);
    std::fill(h_block_table_, h_block_table_ + static_cast<size_t>(capacity_) * stride_, -1);
    (void)hipMemcpy(d_all_, h_all_, all, hipMemcpyHostToDevice);
}

DecodeBatch::~DecodeBatch() { release(); }

void DecodeBatch::release()
{
    if (d_all_) (void)hipFree(d_all_);
    if (h_all_) (void)hipHostFree(h_all_);
    d_all_ = h_all_ = h_dev_ = d_block_table_ = d_context_lens_ = h_block_table_ = h_context_lens_ = nullptr;
}

int DecodeBatch::pack(const std::vector<const GenerationRequest*>& requests)
{
    if (!ok() || static_cast<int>(requests.size()) > capacity_) return -1;
    int width = 1;
    for (const GenerationRequest* r : requests)
    {
        if (r == nullptr || static_cast<int>(r->block_table.size()) > stride_) return -1;
        width = std::max(width, static_cast<int>(r->block_table.size()));
    }
    for (int i = 0; i < capacity_; ++i)
    {
        int32_t* row = h_block_table_ + static_cast<size_t>(i) * stride_;
        if (i < static_cast<int>(requests.size()))
        {
            const GenerationRequest* r = requests[i];
            h_context_lens_[i] = r->context_len;
            const int n = static_cast<int>(r->block_table.size());
            std::copy(r->block_table.begin(), r->block_table.end(), row);
            std::fill(row + n, row + width, -1);
        }
        else
        {
            h_context_lens_[i] = 0;
            std::fill(row, row + width, -1);
        }
    }
    rows_ = static_cast<int>(requests.size());
    width_ = width;
    return width;
}

bool DecodeBatch::upload(hipStream_t stream)
{
    if (!ok()) return false;
    // one copy over rows [0, lens_rows + capacity) of the combined buffer: every row's first w ints, w covering
    // the context lengths (capacity ints in row 0, or whole rows when they take several) and the live width
    const size_t rows = static_cast<size_t>(lens_rows_) + static_cast<size_t>(capacity_);
    const int    w = std::max(width_, lens_rows_ == 1 ? capacity_ : stride_);
    const size_t pitch = static_cast<size_t>(stride_) * sizeof(int32_t);
    hipError_t   e;
    if (h_dev_ != nullptr)  // one kernel reads the mapped staging: a launch instead of a DMA transfer's start-up
        e = ffkv::launch_staging_copy(d_all_, h_dev_, stride_, std::min(w, stride_), static_cast<int>(rows), stream);
    else if (w >= stride_)
        e = hipMemcpyAsync(d_all_, h_all_, rows * pitch, hipMemcpyHostToDevice, stream);
    else
        e = hipMemcpy2DAsync(d_all_, pitch, h_all_, pitch, static_cast<size_t>(w) * sizeof(int32_t), rows,
                             hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return false;
    last_bytes_ = rows * static_cast<size_t>(std::min(w, stride_)) * sizeof(int32_t);
    return true;
}

namespace hal
{

Graph::~Graph() { destroy(); }

Graph::Graph(Graph&& other) noexcept : graph_(other.graph_), exec_(other.exec_)
{
    other.graph_ = nullptr;
    other.exec_ = nullptr;
}

Graph& Graph::operator=(Graph&& other) noexcept
{
    if (this != &other)
    {
        destroy();
        graph_ = std::exchange(other.graph_, nullptr);
        exec_ = std::exchange(other.exec_, nullptr);
    }
    return *this;
}

void Graph::destroy()
{
    if (exec_) (void)hipGraphExecDestroy(exec_);
    if (graph_) (void)hipGraphDestroy(graph_);
    exec_ = nullptr;
    graph_ = nullptr;
}

namespace
{
Status hip_error(hipError_t e, const char* what) { return unexpected(Error{e, what}); }
Status runtime_error(std::string msg) { return unexpected(Error{-1, ErrorCategory::Runtime, msg}); }
}  // namespace

Status Graph::capture(hipStream_t stream, std::function<void()> func)
{
    destroy();
    hipError_t e = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_error(e, "hipStreamBeginCapture");
    // fn may throw: the capture is ended (and its partial graph dropped) before the error is returned
    std::string thrown;
    try
    {
        func();
    }
    catch (const std::exception& ex)
    {
        thrown = std::string("exception during graph capture: ") + ex.what();
    }
    catch (...)
    {
        thrown = "unknown exception during graph capture";
    }
    e = hipStreamEndCapture(stream, &graph_);
    if (!thrown.empty())
    {
        destroy();
        return runtime_error(thrown);
    }
    if (e != hipSuccess)
    {
        destroy();
        return hip_error(e, "hipStreamEndCapture");
    }
    e = hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0);
    if (e != hipSuccess)
    {
        destroy();
        return hip_error(e, "hipGraphInstantiate");
    }
    return {};
}

Status Graph::launch(hipStream_t stream) const
{
    if (!exec_) return runtime_error("Graph: nothing captured to launch");
    const hipError_t e = hipGraphLaunch(exec_, stream);
    if (e != hipSuccess) return hip_error(e, "hipGraphLaunch");
    return {};
}

}  // namespace hal

}  // namespace firefly
