// decode_batch.h - host packing of a decode step's block tables and context lengths (MI355X).
//
// Replaces the per-step packing of the reference engine (src/engine.cc:296-323 with GraphData,
// include/firefly/engine.h:56-68): pinned host staging filled from the scheduled requests, then copied to the
// fixed device buffers a captured decode graph reads.  The reference fills a [bs, max_context_blocks] table whose
// row stride is the POOL size (src/engine.cc:96,126,310) and copies all of it, and the context lengths, in
// separate copies every step (25.6 MB at 64 x 100k blocks); here the device table keeps a fixed row stride (so a
// graph captured once stays valid) and each upload is ONE copy: the context lengths sit in the rows just before
// the table in one buffer of that row stride (host and device alike), and the copy takes only the live width of
// every row (the longest row's block count, at least the lengths' width): one small kernel that reads the pinned
// staging through its device mapping (a launch, where a DMA copy costs about 10 us of start-up), or, where the
// staging has no device mapping, a plain copy when that width is the whole stride and a 2D copy otherwise.
// Entries beyond a row's live blocks are never read by the path's kernels (they
// read blocks 0 .. ceil((context_len + new tokens) / 16) - 1 of a row), so stale device entries there are
// harmless.
//
// Padding rows (batch slots past the live requests) get context_len 0 and block -1, as in the reference
// (src/engine.cc:298-300): append skips them and decode gives them zeros.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "firefly/request.h"
#include "firefly/types.h"

namespace firefly
{

class FIREFLY_API DecodeBatch
{
public:
    /**
     * @param batch_capacity      slots (the graph's batch size)
     * @param max_context_blocks  row stride of the device block table (blocks a row may reach)
     */
    DecodeBatch(int batch_capacity, int max_context_blocks);
    ~DecodeBatch();
    DecodeBatch(const DecodeBatch&) = delete;
    DecodeBatch& operator=(const DecodeBatch&) = delete;

    /// Fill the pinned staging from the requests (at most batch_capacity; their block_table and context_len),
    /// padding the other slots.  Returns the live width in blocks, or -1 if a request does not fit (more requests
    /// than slots, or a block table longer than max_context_blocks).
    int pack(const std::vector<const GenerationRequest*>& requests);

    /// Copy the packed context lengths and the live width of every table row to the device, on `stream`, as one
    /// copy (a kernel reading the mapped staging).  Asynchronous; the staging must not be re-packed until the copy
    /// has completed on the stream.
    bool upload(hipStream_t stream);

    const int32_t* device_context_lens() const { return d_context_lens_; }
    const int32_t* device_block_table() const { return d_block_table_; }
    int32_t*       host_context_lens() { return h_context_lens_; }
    int32_t*       host_block_table() { return h_block_table_; }
    int            batch_capacity() const { return capacity_; }
    int            stride() const { return stride_; }   ///< row stride of the device table (max_context_blocks)
    int            live_rows() const { return rows_; }  ///< requests packed by the last pack()
    int            live_width() const { return width_; }
    size_t         last_upload_bytes() const { return last_bytes_; }
    bool           ok() const { return d_block_table_ != nullptr && h_block_table_ != nullptr; }

private:
    void release();

    int      capacity_ = 0;
    int      stride_ = 0;
    int      rows_ = 0;
    int      width_ = 1;
    size_t   last_bytes_ = 0;
    int      lens_rows_ = 1;             // rows of `stride` ints holding the context lengths
    int32_t* h_all_ = nullptr;           // pinned [lens_rows + capacity, stride]: context lengths, then the table
    int32_t* d_all_ = nullptr;           // the same on the device
    int32_t* h_dev_ = nullptr;           // h_all_'s address on the device (mapped), read by the upload kernel
    int32_t* h_context_lens_ = nullptr;  // = h_all_
    int32_t* h_block_table_ = nullptr;   // = h_all_ + lens_rows * stride, [capacity, stride]
    int32_t* d_context_lens_ = nullptr;
    int32_t* d_block_table_ = nullptr;
};

}  // namespace firefly
