// allocator.h - device memory for tensors.
//
// Same interface as the reference's DeviceAllocator (include/firefly/mm/allocator.h:9-33).  The GPU side is
// stream-ordered (hipMallocAsync / hipFreeAsync on a thread-local default stream, like the reference's
// cudaMallocAsync, src/allocator_cuda.cu:44-68) so tensors created inside hipGraph capture become graph memory
// nodes.  init() raises the pool's release threshold so freed blocks stay cached (src/allocator_cuda.cu:14-42).
#pragma once

#include <cstddef>
#include <cstdint>

#include "firefly/types.h"

namespace firefly
{

template <Device D>
struct DeviceAllocator;

template <>
struct FIREFLY_API DeviceAllocator<Device::CPU>
{
    static void* allocate(size_t bytes);
    static void  free(void* ptr);
};

template <>
struct FIREFLY_API DeviceAllocator<Device::GPU>
{
    // device_id -1 = current device; release_threshold_bytes = bytes the pool keeps cached after frees.
    static void init(int device_id = -1, size_t release_threshold_bytes = UINT64_MAX);

    // Stream used by allocate/free on the calling thread (nullptr = the null stream).
    static void  set_default_stream(void* stream);
    static void* get_default_stream();

    static void* allocate(size_t bytes, void* stream = nullptr);
    static void  free(void* ptr, void* stream = nullptr);
};

}  // namespace firefly
