// kv_append.hip - scatter new K/V tokens into block-table-addressed KV pages on gfx950.
//
// Replaces the reference's append kernel (src/model/qwen_model.cu:21-47), which runs one 128-thread block per
// (token, kv_head, sequence) and stores one 2-byte element per thread.  Here a (token, kv_head) row of
// head_dim elements is handled by head_dim/8 lanes, each moving one 8-element chunk (16 B for 16-bit data) with
// a single vector load and store.  All kv heads of a token are contiguous in both the source [B, S, Hkv, D] and
// the page [N, 16, Hkv, D], so consecutive lanes stream contiguous bytes; a 256-thread workgroup strides over
// rows, two per lane in flight.  Quantizing caches compute the per-row int8 scale with a cross-lane max inside the
// row's lane group.
#include "ffkv_device.h"
#include "ffkv_internal.h"

namespace ffkv
{

// Quantize or convert one lane's 8 elements of a (token, head) row for the cache and store them; int8 also writes
// the row's scale (lane 0 of the row).  LPR lanes hold a row; the cross-lane absmax stays inside them.
// fp8: head_scale is the row's kv-head scale (loaded by the caller with the row's addressing).
// act: the lane holds dims of the row (lanes past head_dim / 8 take part in the int8 max with zeros, store nothing).
template <int SRC, int CACHE, int LPR>
__device__ __forceinline__ void put_row8(const Raw8& raw, void* cache, size_t dst, float* scale_out, size_t dst_row,
                                         float head_scale, int lane, bool act)
{
    if constexpr (SRC == CACHE)
    {
        if (act) store_raw8<CACHE>(cache, dst, raw);
    }
    else
    {
        float x[8];
        unpack8<SRC>(raw, x);
        Raw8 out;
        if constexpr (CACHE == I8 || CACHE == FP8)
        {
            float sc;
            if constexpr (CACHE == I8)
            {
                float amax = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i)
                {
                    const float v = __builtin_fabsf(x[i]);
                    amax = v > amax ? v : amax;  // NaN never compares greater: ignored
                }
                amax = group_max<LPR>(amax);
                sc = amax / 127.0f;
                if (lane == 0) scale_out[dst_row] = amax == 0.0f ? 0.0f : sc;
                if (amax == 0.0f) sc = 1.0f;  // an all-zero row gives codes 0 either way
            }
            else
            {
                sc = head_scale;
            }
            quant8<CACHE == I8>(x, sc, out.w);
        }
        else
        {
            pack8<CACHE>(x, out);
        }
        if (act) store_raw8<CACHE>(cache, dst, out);
    }
}

// DT: head_dim, or 0 for a runtime head_dim (a multiple of 8 up to 8 * LPR); LPR: lanes per row (a power of two,
// DT / 8 when DT is given).  IDX: the row-index type, 32-bit when batch * seq_len * num_kv_heads fits (divisions
// by the head and token counts are then 32-bit), 64-bit otherwise.  A workgroup iteration covers U groups of RPI consecutive rows; a
// lane takes one row of each group.  Its loads go out in dependency order: the addressing chain (context length,
// then block-table entry, and for fp8 the head scales) before the source rows, so the wait for the table entries
// does not also wait for the source rows.
#ifndef FFKV_APPEND_U
#define FFKV_APPEND_U 2  // row groups per workgroup iteration (rows in flight per lane)
#endif

template <int SRC, int CACHE, int DT, int LPR, typename IDX>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a)
{
    static_assert(DT == 0 || DT == 8 * LPR, "a given head_dim has head_dim / 8 lanes per row");
    constexpr int RPI = 256 / LPR;  // rows per group
    constexpr int U = FFKV_APPEND_U;
    const int     D = DT != 0 ? DT : a.head_dim;
    const int     lane = threadIdx.x % LPR;
    const bool    act = DT != 0 || lane * 8 < D;
    const IDX     rows = static_cast<IDX>(a.batch) * static_cast<IDX>(a.seq_len) * static_cast<IDX>(a.num_kv_heads);
    const IDX     step = static_cast<IDX>(gridDim.x) * (RPI * U);
    const IDX     hkv = static_cast<IDX>(a.num_kv_heads), sl = static_cast<IDX>(a.seq_len);

    for (IDX base = static_cast<IDX>(blockIdx.x) * (RPI * U) + threadIdx.x / LPR; base < rows; base += step)
    {
        Raw8    kr[U], vr[U];
        int     h[U], b[U], t[U];
        int64_t pos[U];
        bool    live[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            const IDX r = base + static_cast<IDX>(u * RPI);
            live[u] = r < rows;
            const IDX rr = live[u] ? r : 0;
            const IDX bt = rr / hkv;
            h[u] = static_cast<int>(rr - bt * hkv);
            const IDX bb = bt / sl;
            t[u] = static_cast<int>(bt - bb * sl);
            b[u] = static_cast<int>(bb);
        }
        // pos = context_lens[b] + t; page = block_table[b, pos/16]; slot = pos % 16  (qwen_model.cu:32-37)
#pragma unroll
        for (int u = 0; u < U; ++u) pos[u] = static_cast<int64_t>(a.context_lens ? a.context_lens[b[u]] : 0) + t[u];
        float ksc[U], vsc[U];  // fp8: the rows' kv-head scales
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            ksc[u] = vsc[u] = 1.0f;
            if constexpr (CACHE == FP8)
            {
                ksc[u] = a.k_scale[h[u]];
                vsc[u] = a.v_scale[h[u]];
            }
        }
        int phys[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            phys[u] = -1;
            if (live[u] && pos[u] >= 0 && (pos[u] >> 4) < a.max_blocks)
                phys[u] = a.block_table[static_cast<int64_t>(b[u]) * a.max_blocks + (pos[u] >> 4)];
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            if (live[u] && act)
            {
                const size_t src = static_cast<size_t>(base + static_cast<IDX>(u * RPI)) * D + lane * 8;  // :39
                load_raw8<SRC>(a.k_src, src, kr[u]);
                load_raw8<SRC>(a.v_src, src, vr[u]);
            }
            else
            {
                kr[u] = Raw8{};
                vr[u] = Raw8{};
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            // skipped rows are skipped by all their lanes, the only ones an int8 row's cross-lane max reads
            if (phys[u] < 0 || phys[u] >= a.num_blocks) continue;
            const size_t dst_row =
                (static_cast<size_t>(phys[u]) * kBlockSize + (pos[u] & 15)) * a.num_kv_heads + h[u];
            const size_t dst = dst_row * D + lane * 8;  // qwen_model.cu:41-42
            put_row8<SRC, CACHE, LPR>(kr[u], a.k_cache, dst, a.k_scale, dst_row, ksc[u], lane, act);
            put_row8<SRC, CACHE, LPR>(vr[u], a.v_cache, dst, a.v_scale, dst_row, vsc[u], lane, act);
        }
    }
}

namespace
{

template <int SRC, int CACHE, typename IDX>
void launch_i(const AppendArgs& a, int64_t rows, hipStream_t stream)
{
    auto grid_for = [&](int rows_per_iter)
    {
        int64_t g = (rows + rows_per_iter - 1) / rows_per_iter;
        return static_cast<unsigned>(g < 8192 ? g : 8192);
    };
    switch (a.head_dim)
    {
        case 64:
            hipLaunchKernelGGL((append_kernel<SRC, CACHE, 64, 8, IDX>), dim3(grid_for(32 * FFKV_APPEND_U)), dim3(256),
                               0, stream, a);
            break;
        case 128:
            hipLaunchKernelGGL((append_kernel<SRC, CACHE, 128, 16, IDX>), dim3(grid_for(16 * FFKV_APPEND_U)),
                               dim3(256), 0, stream, a);
            break;
        case 256:
            hipLaunchKernelGGL((append_kernel<SRC, CACHE, 256, 32, IDX>), dim3(grid_for(8 * FFKV_APPEND_U)), dim3(256),
                               0, stream, a);
            break;
        default:  // any other multiple of 8 up to 128: 16 lanes per row, those past head_dim / 8 idle
            hipLaunchKernelGGL((append_kernel<SRC, CACHE, 0, 16, IDX>), dim3(grid_for(16 * FFKV_APPEND_U)), dim3(256),
                               0, stream, a);
            break;
    }
}

template <int SRC, int CACHE>
hipError_t launch_d(const AppendArgs& a, hipStream_t stream)
{
    const int64_t rows = static_cast<int64_t>(a.batch) * a.seq_len * a.num_kv_heads;
    // 32-bit indices while the last row index plus a grid stride cannot wrap
    if (rows < (int64_t{1} << 31))
        launch_i<SRC, CACHE, uint32_t>(a, rows, stream);
    else
        launch_i<SRC, CACHE, uint64_t>(a, rows, stream);
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
