// rope_append.hip - rotary position embedding of q and k, fused with the KV-page append, on gfx950.
//
// Replaces the reference's rope_kernel_optimized (src/kernels/rope.cu:22-137) followed by its append kernel
// (src/model/qwen_model.cu:21-47, launched at :138-143 right after kernels::apply_rope at :136).  Semantics
// (rotate-half form, src/kernels/rope.cu:62-91): for token t of sequence b at position pos = context_lens[b] + t
// (t when context_lens is null, :37), pair i of a head (dims i and i + D/2, 0 <= i < D/2) is rotated by
// angle = pos * inv_freq_i:
//     lo' = lo * cos - hi * sin,   hi' = hi * cos + lo * sin
// q and k are rotated in place in their own dtype, then k (as rotated and rounded) and v are appended to the
// pages exactly as the append kernel does, quantizing for int8/fp8 caches.
//
// Arithmetic, chosen so a CPU restatement reproduces it bit for bit: inv_freq_i = float(theta^(-2i/D)) and
// cos/sin = float(cos/sin(double(angle))) are evaluated in double precision and rounded once to fp32;
// angle = float(pos) * inv_freq_i is one fp32 product; the rotation is two fp32 products and one fp32 sum each,
// without fused multiply-add, then rounded to the tensor dtype.  (The reference computes the same quantities
// with fast-math powf/cosf/sinf, whose error grows with the angle; it is not bit-reproducible.)
//
// Layout: a workgroup of 256 threads takes 256 / (D/2) tokens per iteration (grid-stride): each thread computes
// one (cos, sin) pair of one of them into LDS (inv_freq once per thread, outside the loop), and the tokens' Hq +
// Hkv head rows are spread over the workgroup, D/16 lanes per row, each lane holding 8 dims of the low half and
// the matching 8 dims of the high half.  A thread issues the loads of two rows before rotating either, and the
// first two rows' loads go out before the table's barrier, so the loads overlap the double-precision sin/cos.
#include "ffkv_device.h"
#include "ffkv_internal.h"

namespace ffkv
{

#ifndef FFKV_ROPE_NB
#define FFKV_ROPE_NB 1
#endif

namespace
{

__device__ __forceinline__ float rot_lo(float lo, float hi, float c, float s)
{
#pragma clang fp contract(off)
    return lo * c - hi * s;
}

__device__ __forceinline__ float rot_hi(float lo, float hi, float c, float s)
{
#pragma clang fp contract(off)
    return hi * c + lo * s;
}

// Write 8 values of a (token, head) row to the cache at element index dst.  int8: sc = row absmax / 127, or 0
// for an all-zero row; fp8: sc = the head's scale.
template <int CACHE>
__device__ __forceinline__ void store_cache8(void* cache, size_t dst, const float* x, float sc)
{
    Raw8 out;
    if constexpr (CACHE == I8)
    {
        quant8<true>(x, sc == 0.0f ? 1.0f : sc, out.w);
        if (sc == 0.0f) out.w[0] = out.w[1] = 0u;  // an all-zero row
    }
    else if constexpr (CACHE == FP8)
    {
        quant8<false>(x, sc, out.w);
    }
    else
    {
        pack8<CACHE>(x, out);
    }
    store_raw8<CACHE>(cache, dst, out);
}

// Append one (token, kv head) row given as two 8-value chunks per lane (dims 8*lane.. and D/2 + 8*lane..) of
// LPR lanes.  int8 caches write the row scale from lane 0 of the row.
template <int CACHE, int D, int LPR>
__device__ __forceinline__ void append_row(void* cache, float* scales, int h, size_t dst_row, int lane, const float* xl,
                                           const float* xh)
{
    float sc = 0.0f;
    if constexpr (CACHE == I8)
    {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            const float u = __builtin_fabsf(xl[i]);
            const float w = __builtin_fabsf(xh[i]);
            amax = u > amax ? u : amax;  // NaN never compares greater: ignored
            amax = w > amax ? w : amax;
        }
        amax = group_max<LPR>(amax);
        sc = amax == 0.0f ? 0.0f : amax / 127.0f;
        if (lane == 0) scales[dst_row] = sc;
    }
    else if constexpr (CACHE == FP8)
    {
        sc = scales[h];
    }
    store_cache8<CACHE>(cache, dst_row * D + 8 * lane, xl, sc);
    store_cache8<CACHE>(cache, dst_row * D + D / 2 + 8 * lane, xh, sc);
}

}  // namespace

// TPI tokens per iteration: 256 / (D/2) for bulk calls (every thread computes one (cos, sin) pair), 1 for
// small calls, which then spread over more workgroups.
template <int SRC, int CACHE, int D, bool APPEND, int TPI>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeArgs a)
{
    constexpr int HALF = D / 2;
    constexpr int LPR = D / 16;     // lanes per head row
    constexpr int RPP = 256 / LPR;  // head rows per pass of the workgroup
    constexpr int NB = FFKV_ROPE_NB; // rows per thread whose loads are issued before any of them is rotated
    __shared__ float s_cos[TPI][HALF], s_sin[TPI][HALF];

    const int     lane = threadIdx.x % LPR;
    const int     rsub = threadIdx.x / LPR;
    const int64_t tokens = static_cast<int64_t>(a.batch) * a.seq_len;
    const int     rows = a.num_heads + a.num_kv_heads;  // head rows of one token
    const int     iter_rows = TPI * rows;

    // inv_freq of this thread's pair, once (:74-76)
    const int   my_i = threadIdx.x % HALF;
    const int   my_t = threadIdx.x / HALF;  // table row this thread fills (threads beyond TPI rows fill none)
    const float inv_freq = static_cast<float>(pow(static_cast<double>(a.theta), -2.0 * my_i / D));

    for (int64_t tok0 = static_cast<int64_t>(blockIdx.x) * TPI; tok0 < tokens; tok0 += static_cast<int64_t>(gridDim.x) * TPI)
    {
        __syncthreads();  // the previous tokens' rows are done with the table
        {
            const int64_t tok = tok0 + my_t;
            if (my_t < TPI && tok < tokens)
            {
                const int     b = static_cast<int>(tok / a.seq_len);
                const int     t = static_cast<int>(tok % a.seq_len);
                const int64_t pos = static_cast<int64_t>(a.context_lens ? a.context_lens[b] : 0) + t;  // :36-37
                const float   ang = static_cast<float>(pos) * inv_freq;                                // :77
                s_cos[my_t][my_i] = static_cast<float>(cos(static_cast<double>(ang)));
                s_sin[my_t][my_i] = static_cast<float>(sin(static_cast<double>(ang)));
            }
        }

        // Row u of the iteration: token tok0 + u / rows, head row u % rows (q heads, then kv heads).  Loads of NB
        // rows go out first (before the table barrier for the first batch), then the rows are rotated and stored.
        // every thread runs the first batch (possibly without rows) so that all reach the table barrier
        for (int u0 = rsub;; u0 += NB * RPP)
        {
            Raw8 rl[NB], rh[NB], vl[NB], vh[NB];
            bool act[NB], isq[NB];
            int  tl[NB], hh[NB];
            size_t rowoff[NB];
#pragma unroll
            for (int k = 0; k < NB; ++k)
            {
                const int     u = u0 + k * RPP;
                const int     tli = u / rows;
                const int64_t tok = tok0 + tli;
                act[k] = u < iter_rows && tok < tokens;
                tl[k] = tli;
                const int hr = u % rows;
                isq[k] = hr < a.num_heads;
                hh[k] = isq[k] ? hr : hr - a.num_heads;
                rowoff[k] = (static_cast<size_t>(act[k] ? tok : 0) * (isq[k] ? a.num_heads : a.num_kv_heads) + hh[k]) * D;
                if (act[k])
                {
                    const void* base = isq[k] ? a.q : a.k;
                    load_raw8<SRC>(base, rowoff[k] + 8 * lane, rl[k]);
                    load_raw8<SRC>(base, rowoff[k] + HALF + 8 * lane, rh[k]);
                    if constexpr (APPEND)
                    {
                        if (!isq[k])
                        {
                            load_raw8<SRC>(a.v, rowoff[k] + 8 * lane, vl[k]);
                            load_raw8<SRC>(a.v, rowoff[k] + HALF + 8 * lane, vh[k]);
                        }
                    }
                }
            }
            if (u0 == rsub) __syncthreads();  // the table of these tokens is written (first batch: every thread)
#pragma unroll
            for (int k = 0; k < NB; ++k)
            {
                if (!act[k]) continue;
                float xl[8], xh[8], yl[8], yh[8];
                unpack8<SRC>(rl[k], xl);
                unpack8<SRC>(rh[k], xh);
#pragma unroll
                for (int e = 0; e < 8; ++e)
                {
                    const float c = s_cos[tl[k]][8 * lane + e];
                    const float s = s_sin[tl[k]][8 * lane + e];
                    yl[e] = rot_lo(xl[e], xh[e], c, s);
                    yh[e] = rot_hi(xl[e], xh[e], c, s);
                }
                pack8<SRC>(yl, rl[k]);
                pack8<SRC>(yh, rh[k]);
                void* base = isq[k] ? a.q : a.k;
                store_raw8<SRC>(base, rowoff[k] + 8 * lane, rl[k]);
                store_raw8<SRC>(base, rowoff[k] + HALF + 8 * lane, rh[k]);

                if constexpr (APPEND)
                {
                    if (isq[k]) continue;
                    // page slot of the row's token, as the append kernel computes it
                    const int64_t tok = tok0 + tl[k];
                    const int     b = static_cast<int>(tok / a.seq_len);
                    const int     t = static_cast<int>(tok % a.seq_len);
                    const int64_t pos = static_cast<int64_t>(a.context_lens ? a.context_lens[b] : 0) + t;
                    bool          ok = pos >= 0 && (pos >> 4) < a.max_blocks;
                    int           phys = -1;
                    if (ok)
                    {
                        phys = a.block_table[static_cast<int64_t>(b) * a.max_blocks + (pos >> 4)];
                        ok = phys >= 0 && phys < a.num_blocks;
                    }
                    // `ok` is per token, the same for the row's LPR lanes (the only ones the int8 reduction reads)
                    if (!ok) continue;
                    const int    h = hh[k];
                    const size_t dst_row = (static_cast<size_t>(phys) * kBlockSize + (pos & 15)) * a.num_kv_heads + h;
                    // k as stored in its dtype (the values the reference's append would read back)
                    unpack8<SRC>(rl[k], yl);
                    unpack8<SRC>(rh[k], yh);
                    if constexpr (SRC == CACHE)
                    {
                        store_raw8<CACHE>(a.k_cache, dst_row * D + 8 * lane, rl[k]);
                        store_raw8<CACHE>(a.k_cache, dst_row * D + HALF + 8 * lane, rh[k]);
                        store_raw8<CACHE>(a.v_cache, dst_row * D + 8 * lane, vl[k]);
                        store_raw8<CACHE>(a.v_cache, dst_row * D + HALF + 8 * lane, vh[k]);
                    }
                    else
                    {
                        append_row<CACHE, D, LPR>(a.k_cache, a.k_scale, h, dst_row, lane, yl, yh);
                        unpack8<SRC>(vl[k], xl);
                        unpack8<SRC>(vh[k], xh);
                        append_row<CACHE, D, LPR>(a.v_cache, a.v_scale, h, dst_row, lane, xl, xh);
                    }
                }
            }
            if (u0 + NB * RPP >= iter_rows) break;
        }
    }
}

namespace
{

template <int SRC, int CACHE, bool APPEND, int D>
hipError_t launch_ra_t(const RopeArgs& a, hipStream_t stream)
{
    constexpr int64_t kBulk = 256 / (D / 2);
    const int64_t     tokens = static_cast<int64_t>(a.batch) * a.seq_len;
    const bool        bulk = tokens >= 2048;  // small calls: one token per workgroup iteration, more workgroups
    const int64_t     tpi = bulk ? kBulk : 1;
    const int64_t     iters = (tokens + tpi - 1) / tpi;
    const auto        grid = dim3(static_cast<unsigned>(iters < 16384 ? iters : 16384));
    if (bulk)
        hipLaunchKernelGGL((rope_append_kernel<SRC, CACHE, D, APPEND, kBulk>), grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((rope_append_kernel<SRC, CACHE, D, APPEND, 1>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <int SRC, int CACHE, bool APPEND>
hipError_t launch_ra_d(const RopeArgs& a, hipStream_t stream)
{
    switch (a.head_dim)
    {
        case 64:
            return launch_ra_t<SRC, CACHE, APPEND, 64>(a, stream);
        case 128:
            return launch_ra_t<SRC, CACHE, APPEND, 128>(a, stream);
        default:
            return launch_ra_t<SRC, CACHE, APPEND, 256>(a, stream);
    }
}

template <int SRC>
hipError_t launch_ra_c(const RopeArgs& a, hipStream_t stream)
{
    if (a.k_cache == nullptr) return launch_ra_d<SRC, SRC, false>(a, stream);
    switch (a.cache_dtype)
    {
        case F32:
            return launch_ra_d<SRC, F32, true>(a, stream);
        case F16:
            return launch_ra_d<SRC, F16, true>(a, stream);
        case BF16:
            return launch_ra_d<SRC, BF16, true>(a, stream);
        case I8:
            return launch_ra_d<SRC, I8, true>(a, stream);
        default:
            return launch_ra_d<SRC, FP8, true>(a, stream);
    }
}

}  // namespace

hipError_t launch_rope_append(const RopeArgs& a, hipStream_t stream)
{
    switch (a.src_dtype)
    {
        case F32:
            return launch_ra_c<F32>(a, stream);
        case F16:
            return launch_ra_c<F16>(a, stream);
        default:
            return launch_ra_c<BF16>(a, stream);
    }
}

}  // namespace ffkv
