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
// Layout: one workgroup per token (grid-stride over tokens).  The D/2 (cos, sin) pairs of the token are
// computed once into LDS, then its Hq + Hkv head rows are spread over the workgroup, D/16 lanes per row, each
// lane holding 8 dims of the low half and the matching 8 dims of the high half.
#include "ffkv_device.h"
#include "ffkv_internal.h"

namespace ffkv
{

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
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = sc == 0.0f ? 0u : (quant_i8(x[i], sc) & 0xffu);
        out.w[0] = q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24);
        out.w[1] = q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24);
    }
    else if constexpr (CACHE == FP8)
    {
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = f32_to_e4m3(x[i] / sc);
        out.w[0] = q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24);
        out.w[1] = q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24);
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
#pragma unroll
        for (int off = 1; off < LPR; off <<= 1)
        {
            const float o = __shfl_xor(amax, off, 64);
            amax = o > amax ? o : amax;
        }
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

template <int SRC, int CACHE, int D, bool APPEND>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeArgs a)
{
    constexpr int HALF = D / 2;
    constexpr int LPR = D / 16;      // lanes per head row
    constexpr int RPP = 256 / LPR;   // head rows per pass of the workgroup
    __shared__ float s_cos[HALF], s_sin[HALF];

    const int     lane = threadIdx.x % LPR;
    const int     rsub = threadIdx.x / LPR;
    const int64_t tokens = static_cast<int64_t>(a.batch) * a.seq_len;
    const int     rows = a.num_heads + a.num_kv_heads;

    for (int64_t tok = blockIdx.x; tok < tokens; tok += gridDim.x)
    {
        const int     b = static_cast<int>(tok / a.seq_len);
        const int     t = static_cast<int>(tok % a.seq_len);
        const int64_t pos = static_cast<int64_t>(a.context_lens ? a.context_lens[b] : 0) + t;  // rope.cu:36-37

        __syncthreads();  // the previous token's rows are done with the table
        if (threadIdx.x < HALF)
        {
            const int   i = threadIdx.x;
            const float inv_freq = static_cast<float>(pow(static_cast<double>(a.theta), -2.0 * i / D));  // :74-76
            const float ang = static_cast<float>(pos) * inv_freq;                                          // :77
            s_cos[i] = static_cast<float>(cos(static_cast<double>(ang)));
            s_sin[i] = static_cast<float>(sin(static_cast<double>(ang)));
        }
        __syncthreads();

        // Page slot of this token (uniform over the workgroup), as the append kernel computes it.
        bool   ok = false;
        size_t slot_row = 0;  // (phys * 16 + pos % 16) * Hkv
        if constexpr (APPEND)
        {
            ok = pos >= 0 && (pos >> 4) < a.max_blocks;
            if (ok)
            {
                const int phys = a.block_table[static_cast<int64_t>(b) * a.max_blocks + (pos >> 4)];
                ok = phys >= 0 && phys < a.num_blocks;
                slot_row = (static_cast<size_t>(phys) * kBlockSize + (pos & 15)) * a.num_kv_heads;
            }
        }

        for (int u = rsub; u < rows; u += RPP)
        {
            const bool   is_q = u < a.num_heads;
            const int    h = is_q ? u : u - a.num_heads;
            void*        base = is_q ? a.q : a.k;
            const size_t row = (static_cast<size_t>(tok) * (is_q ? a.num_heads : a.num_kv_heads) + h) * D;
            Raw8         rl, rh;
            load_raw8<SRC>(base, row + 8 * lane, rl);
            load_raw8<SRC>(base, row + HALF + 8 * lane, rh);
            float xl[8], xh[8], yl[8], yh[8];
            unpack8<SRC>(rl, xl);
            unpack8<SRC>(rh, xh);
#pragma unroll
            for (int e = 0; e < 8; ++e)
            {
                const float c = s_cos[8 * lane + e];
                const float s = s_sin[8 * lane + e];
                yl[e] = rot_lo(xl[e], xh[e], c, s);
                yh[e] = rot_hi(xl[e], xh[e], c, s);
            }
            pack8<SRC>(yl, rl);
            pack8<SRC>(yh, rh);
            store_raw8<SRC>(base, row + 8 * lane, rl);
            store_raw8<SRC>(base, row + HALF + 8 * lane, rh);

            if constexpr (APPEND)
            {
                // `ok` is per token and `is_q` per row: the row's lanes, the only ones the int8 reduction reads,
                // take the same branch.
                if (!is_q && ok)
                {
                    const size_t dst_row = slot_row + h;
                    // k as stored in its dtype (the values the reference's append would read back)
                    unpack8<SRC>(rl, yl);
                    unpack8<SRC>(rh, yh);
                    if constexpr (SRC == CACHE)
                    {
                        store_raw8<CACHE>(a.k_cache, dst_row * D + 8 * lane, rl);
                        store_raw8<CACHE>(a.k_cache, dst_row * D + HALF + 8 * lane, rh);
                    }
                    else
                    {
                        append_row<CACHE, D, LPR>(a.k_cache, a.k_scale, h, dst_row, lane, yl, yh);
                    }
                    Raw8 vl, vh;
                    load_raw8<SRC>(a.v, row + 8 * lane, vl);
                    load_raw8<SRC>(a.v, row + HALF + 8 * lane, vh);
                    if constexpr (SRC == CACHE)
                    {
                        store_raw8<CACHE>(a.v_cache, dst_row * D + 8 * lane, vl);
                        store_raw8<CACHE>(a.v_cache, dst_row * D + HALF + 8 * lane, vh);
                    }
                    else
                    {
                        unpack8<SRC>(vl, xl);
                        unpack8<SRC>(vh, xh);
                        append_row<CACHE, D, LPR>(a.v_cache, a.v_scale, h, dst_row, lane, xl, xh);
                    }
                }
            }
        }
    }
}

namespace
{

template <int SRC, int CACHE, bool APPEND>
hipError_t launch_ra_d(const RopeArgs& a, hipStream_t stream)
{
    const int64_t tokens = static_cast<int64_t>(a.batch) * a.seq_len;
    const auto    grid = dim3(static_cast<unsigned>(tokens < 16384 ? tokens : 16384));
    switch (a.head_dim)
    {
        case 64:
            hipLaunchKernelGGL((rope_append_kernel<SRC, CACHE, 64, APPEND>), grid, dim3(256), 0, stream, a);
            break;
        case 128:
            hipLaunchKernelGGL((rope_append_kernel<SRC, CACHE, 128, APPEND>), grid, dim3(256), 0, stream, a);
            break;
        default:
            hipLaunchKernelGGL((rope_append_kernel<SRC, CACHE, 256, APPEND>), grid, dim3(256), 0, stream, a);
            break;
    }
    return hipGetLastError();
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
