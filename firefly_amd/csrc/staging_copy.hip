// staging_copy.hip - the decode step's upload as a kernel that reads the pinned staging buffer directly.
//
// firefly::DecodeBatch stages each step's context lengths and block tables in pinned host memory mapped into the
// device's address space (hipHostMallocMapped).  A host-to-device hipMemcpyAsync of those few tens of KB costs
// about 10 us on the launch stream, nearly all of it the DMA transfer's own start-up; one small kernel whose
// lanes read the mapped rows over PCIe and store them to the device table takes a kernel launch instead.
#include "ffkv_internal.h"

namespace ffkv
{

namespace
{

// Rows 0 .. rows - 1 of pitch ints each: the first `width` ints of every row (blockIdx.y), 256 per workgroup.
__global__ __launch_bounds__(256) void staging_rows_copy(int32_t* __restrict__ dst, const int32_t* __restrict__ src,
                                                         int pitch, int width, int rows)
{
    const int    r = static_cast<int>(blockIdx.y);
    const int    i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    const size_t o = static_cast<size_t>(r) * static_cast<size_t>(pitch) + static_cast<size_t>(i);
    if (r < rows && i < width) dst[o] = src[o];
}

}  // namespace

hipError_t launch_staging_copy(int32_t* dst, const int32_t* src, int pitch, int width, int rows, hipStream_t stream)
{
    if (rows <= 0 || width <= 0) return hipSuccess;
    if (width > pitch || rows > 65535) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>((width + 255) / 256), static_cast<unsigned>(rows));
    hipLaunchKernelGGL(staging_rows_copy, grid, dim3(256), 0, stream, dst, src, pitch, width, rows);
    return hipGetLastError();
}

}  // namespace ffkv
