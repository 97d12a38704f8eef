// stream_read.hip - a read-only HBM streaming kernel, the practical read ceiling the decode is compared with.
//
// Measurement helper for bench.py only (built into firefly_amd/libffkv_bench.so, not into the product library):
// the paged decode is read-dominated (its algorithmic bytes are ~99.9 % page reads), and a device-to-device copy,
// which moves as many bytes in as out, is not the rate a read stream reaches.  Each workgroup reads contiguous
// 16-byte vectors over a grid-stride loop with UNROLL loads in flight per lane and folds them into one word per
// workgroup (written out so the loads cannot be dropped).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace
{

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

template <int UNROLL>
__global__ __launch_bounds__(256) void stream_read(const u32x4* __restrict__ src, size_t n_vec,
                                                   uint32_t* __restrict__ out)
{
    const size_t stride = static_cast<size_t>(gridDim.x) * 256 * UNROLL;
    size_t       i = static_cast<size_t>(blockIdx.x) * 256 * UNROLL + threadIdx.x;
    u32x4        acc = u32x4{0u, 0u, 0u, 0u};
    for (; i + 256 * (UNROLL - 1) < n_vec; i += stride)
    {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + i + 256 * u);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u];
    }
    for (; i < n_vec; i += 256) acc ^= src[i];
    uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off, 64);
    __shared__ uint32_t s[4];
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = s[0] ^ s[1] ^ s[2] ^ s[3];
}

}  // namespace

// Reads n_bytes (a multiple of 16, 16-byte aligned) from src with `blocks` workgroups of 256 lanes and `unroll`
// (4 or 8) loads in flight per lane; out holds `blocks` words.  Returns 0, or -1 for bad arguments, -4 for a
// launch failure.
extern "C" __attribute__((visibility("default"))) int ffkv_bench_stream_read(const void* src, size_t n_bytes,
                                                                              void* out, int blocks, int unroll,
                                                                              void* stream)
{
    if (src == nullptr || out == nullptr || blocks <= 0 || n_bytes % 16 != 0 || (unroll != 4 && unroll != 8))
        return -1;
    const auto* s = static_cast<const u32x4*>(src);
    auto*       o = static_cast<uint32_t*>(out);
    const auto  st = static_cast<hipStream_t>(stream);
    if (unroll == 4)
        hipLaunchKernelGGL(stream_read<4>, dim3(blocks), dim3(256), 0, st, s, n_bytes / 16, o);
    else
        hipLaunchKernelGGL(stream_read<8>, dim3(blocks), dim3(256), 0, st, s, n_bytes / 16, o);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
