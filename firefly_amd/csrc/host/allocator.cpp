// allocator.cpp - host and stream-ordered device allocation for Tensor.
#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <new>
#include <stdexcept>
#include <string>

#include "firefly/mm/allocator.h"

namespace firefly
{

namespace
{

thread_local void* t_alloc_stream = nullptr;

void hip_check(hipError_t e, const char* what)
{
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

void* DeviceAllocator<Device::CPU>::allocate(size_t bytes)
{
    if (bytes == 0) return nullptr;
    const size_t rounded = (bytes + 63) / 64 * 64;
    void*        p = std::aligned_alloc(64, rounded);
    if (p == nullptr) throw std::bad_alloc();
    return p;
}

void DeviceAllocator<Device::CPU>::free(void* ptr) { std::free(ptr); }

void DeviceAllocator<Device::GPU>::init(int device_id, size_t release_threshold_bytes)
{
    int dev = device_id;
    if (dev < 0) hip_check(hipGetDevice(&dev), "hipGetDevice");
    hipMemPool_t pool;
    hip_check(hipDeviceGetDefaultMemPool(&pool, dev), "hipDeviceGetDefaultMemPool");
    uint64_t threshold = release_threshold_bytes;
    hip_check(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold),
              "hipMemPoolSetAttribute(release threshold)");
}

void DeviceAllocator<Device::GPU>::set_default_stream(void* stream) { t_alloc_stream = stream; }

void* DeviceAllocator<Device::GPU>::get_default_stream() { return t_alloc_stream; }

void* DeviceAllocator<Device::GPU>::allocate(size_t bytes, void* stream)
{
    if (bytes == 0) return nullptr;
    void*      p = nullptr;
    hipError_t e = hipMallocAsync(&p, bytes, static_cast<hipStream_t>(stream ? stream : t_alloc_stream));
    if (e != hipSuccess || p == nullptr)
        throw std::runtime_error("GPU allocation of " + std::to_string(bytes) + " bytes failed: " + hipGetErrorString(e));
    return p;
}

void DeviceAllocator<Device::GPU>::free(void* ptr, void* stream)
{
    if (ptr == nullptr) return;
    (void)hipFreeAsync(ptr, static_cast<hipStream_t>(stream ? stream : t_alloc_stream));
}

}  // namespace firefly
