// kv_append.hip - scatter new K/V tokens into block-table-addressed KV pages on gfx950.
//
// Replaces the reference's append kernel (src/model/qwen_model.cu:21-47), which runs one 128-thread block per
// (token, kv_head, sequence) and stores one 2-byte element per thread.  Here a (token, kv_head) row of
// head_dim elements is handled by head_dim/8 lanes, each moving one 8-element chunk (16 B for 16-bit data) with
// a single vector load and store, and a 256-thread workgroup strides over rows.  All kv heads of a token are
// contiguous in both the source [B, S, Hkv, D] and the page [N, 16, Hkv, D], so consecutive lanes stream
// contiguous bytes.  Quantizing caches compute the per-row int8 scale with a cross-lane max inside the row's
// lane group.
#include "ffkv_device.h"
#include "ffkv_internal.h"

namespace ffkv
{

template <int SRC, int CACHE, int D>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a)
{
    constexpr int LPR = D / 8;      // lanes per (token, head) row
    constexpr int RPI = 256 / LPR;  // rows per workgroup iteration
    const int     lane = threadIdx.x % LPR;
    const int64_t rows = static_cast<int64_t>(a.batch) * a.seq_len * a.num_kv_heads;
    const int64_t step = static_cast<int64_t>(gridDim.x) * RPI;

    for (int64_t r = static_cast<int64_t>(blockIdx.x) * RPI + threadIdx.x / LPR; r < rows; r += step)
    {
        const int     h = static_cast<int>(r % a.num_kv_heads);
        const int64_t bt = r / a.num_kv_heads;
        const int     t = static_cast<int>(bt % a.seq_len);
        const int     b = static_cast<int>(bt / a.seq_len);

        // pos = context_lens[b] + t; page = block_table[b, pos/16]; slot = pos % 16  (qwen_model.cu:32-37)
        const int64_t pos = static_cast<int64_t>(a.context_lens ? a.context_lens[b] : 0) + t;
        bool          ok = pos >= 0 && (pos >> 4) < a.max_blocks;
        int           phys = -1;
        if (ok)
        {
            phys = a.block_table[static_cast<int64_t>(b) * a.max_blocks + (pos >> 4)];
            ok = phys >= 0 && phys < a.num_blocks;
        }
        // `ok` is uniform across the row's lanes, and the row's lanes are the only ones a quantizing
        // cross-lane reduction below reads, so skipping whole rows is safe.
        if (!ok) continue;

        const size_t src = static_cast<size_t>(r) * D + lane * 8;                       // qwen_model.cu:39
        const size_t dst_row = (static_cast<size_t>(phys) * kBlockSize + (pos & 15)) * a.num_kv_heads + h;
        const size_t dst = dst_row * D + lane * 8;                                       // qwen_model.cu:41-42

#pragma unroll
        for (int which = 0; which < 2; ++which)
        {
            const void* s = which ? a.v_src : a.k_src;
            void*       c = which ? a.v_cache : a.k_cache;
            Raw8        raw;
            load_raw8<SRC>(s, src, raw);
            if constexpr (SRC == CACHE)
            {
                store_raw8<CACHE>(c, dst, raw);
            }
            else
            {
                float x[8];
                unpack8<SRC>(raw, x);
                Raw8 out;
                if constexpr (CACHE == I8)
                {
                    float amax = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                    {
                        float v = __builtin_fabsf(x[i]);
                        amax = v > amax ? v : amax;  // NaN never compares greater: ignored
                    }
#pragma unroll
                    for (int off = 1; off < LPR; off <<= 1)
                    {
                        float o = __shfl_xor(amax, off, 64);
                        amax = o > amax ? o : amax;
                    }
                    const float sc = amax / 127.0f;
                    uint32_t    q[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) q[i] = amax == 0.0f ? 0u : (quant_i8(x[i], sc) & 0xffu);
                    out.w[0] = q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24);
                    out.w[1] = q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24);
                    if (lane == 0) (which ? a.v_scale : a.k_scale)[dst_row] = amax == 0.0f ? 0.0f : sc;
                }
                else if constexpr (CACHE == FP8)
                {
                    const float sc = (which ? a.v_scale : a.k_scale)[h];
                    uint32_t    q[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) q[i] = f32_to_e4m3(x[i] / sc);
                    out.w[0] = q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24);
                    out.w[1] = q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24);
                }
                else
                {
                    pack8<CACHE>(x, out);
                }
                store_raw8<CACHE>(c, dst, out);
            }
        }
    }
}

namespace
{

template <int SRC, int CACHE>
hipError_t launch_d(const AppendArgs& a, hipStream_t stream)
{
    const int64_t rows = static_cast<int64_t>(a.batch) * a.seq_len * a.num_kv_heads;
    auto          grid_for = [&](int rpi)
    {
        int64_t g = (rows + rpi - 1) / rpi;
        return static_cast<unsigned>(g < 8192 ? g : 8192);
    };
    switch (a.head_dim)
    {
        case 64:
            hipLaunchKernelGGL((append_kernel<SRC, CACHE, 64>), dim3(grid_for(32)), dim3(256), 0, stream, a);
            break;
        case 128:
            hipLaunchKernelGGL((append_kernel<SRC, CACHE, 128>), dim3(grid_for(16)), dim3(256), 0, stream, a);
            break;
        default:
            hipLaunchKernelGGL((append_kernel<SRC, CACHE, 256>), dim3(grid_for(8)), dim3(256), 0, stream, a);
            break;
    }
    return hipGetLastError();
}

template <int SRC>
hipError_t launch_c(const AppendArgs& a, hipStream_t stream)
{
    switch (a.cache_dtype)
    {
        case F32:
            return launch_d<SRC, F32>(a, stream);
        case F16:
            return launch_d<SRC, F16>(a, stream);
        case BF16:
            return launch_d<SRC, BF16>(a, stream);
        case I8:
            return launch_d<SRC, I8>(a, stream);
        default:
            return launch_d<SRC, FP8>(a, stream);
    }
}

}  // namespace

hipError_t launch_append(const AppendArgs& a, hipStream_t stream)
{
    switch (a.src_dtype)
    {
        case F32:
            return launch_c<F32>(a, stream);
        case F16:
            return launch_c<F16>(a, stream);
        default:
            return launch_c<BF16>(a, stream);
    }
}

}  // namespace ffkv
