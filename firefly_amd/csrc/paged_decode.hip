// paged_decode.hip - PagedAttention decode for gfx950: GQA-shared KV reads, split-K over the context, online
// softmax, and a merge pass.
//
// Reference semantics: paged_attention_kernel (src/kernels/attention.cu:291-447).  The reference runs one
// 128-thread block per (query head, sequence), so every query head of a GQA group re-reads the same KV head, and
// a long context is walked serially by one block.  Here one 256-thread workgroup owns a (chunk, kv_head,
// sequence) work item: it loads the G = Hq/Hkv query vectors of the group once, reads each K/V page slice once
// for all of them, and writes either the final output (rows that fit in one chunk) or an unnormalised partial
// state (m, l, acc) that paged_decode_merge combines.
//
// Lane layout: head_dim/8 lanes per token (one 8-element, 16-byte chunk each for 16-bit KV), so a wave64 covers
// 64/(D/8) tokens per step and the workgroup 256/(D/8).  Head dims other than 64, 128 and 256 (multiples of 8 up
// to 128, which the reference's decode takes) run with 16 lanes per token, those past head_dim/8 idle.  Each token slot keeps its own online-softmax state in
// registers; the slots are merged with cross-lane shuffles inside a wave and through LDS across waves.
// The softmax runs in base 2 with log2(e) folded into the score scale, against a reference maximum that moves only
// when a score passes it by 2^8.  A token's dot product crosses its lanes with DPP steps (no LDS), and each loop
// trip issues the loads of several token groups (and the next trip's block-table entries) before using them: the
// kernel is bound by memory latency, not by its arithmetic.
#include "ffkv_device.h"
#include "ffkv_internal.h"

namespace ffkv
{

namespace
{

#ifndef FFKV_GENERIC_U16
#define FFKV_GENERIC_U16 4
#endif
#ifndef FFKV_GENERIC_U32
#define FFKV_GENERIC_U32 2
#endif

constexpr float kNegBig = -1e30f;  // finite "minus infinity" seed, as in attention.cu:323

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int row_tokens(const DecodeArgs& a, int b)
{
    int64_t L = static_cast<int64_t>(a.context_lens[b]) + 1;  // +1: the token appended this step (:320)
    if (L > a.cap_tokens) L = a.cap_tokens;
    return L < 0 ? 0 : static_cast<int>(L);
}

}  // namespace

// DT: head_dim, or 0 for a runtime head_dim (a multiple of 8 up to 8 * LPT); LPT: lanes per token, a power of two
// (DT / 8 when DT is given).  Lanes past head_dim / 8 hold zeros and store nothing.
template <int CT, int DT, int LPT, int GP>
__global__ __launch_bounds__(256) void paged_decode_generic(DecodeArgs a)
{
    static_assert(DT == 0 || DT == 8 * LPT, "a given head_dim has head_dim / 8 lanes per token");
    constexpr int TPI = 256 / LPT; // token slots per workgroup
    constexpr int WAVES = 4;
    constexpr int DMAX = 8 * LPT;
    const int     D = DT != 0 ? DT : a.head_dim;

    const int chunk_id = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid % LPT;
    const int slot = tid / LPT;
    const int wave = tid / 64;
    const bool act = DT != 0 || lane * 8 < D;  // this lane holds dims of the head

    const int L = row_tokens(a, b);
    const int nch = (L + a.chunk - 1) / a.chunk;
    if (chunk_id >= nch && !(chunk_id == 0 && nch == 0)) return;  // uniform over the workgroup
    const int begin = chunk_id * a.chunk;
    const int end = min(begin + a.chunk, L);
    const int G = a.group;

    float q[GP][8];
#pragma unroll
    for (int g = 0; g < GP; ++g)
    {
        if (g < G && act)
            load_act8(a.q, a.qo_dtype, (static_cast<size_t>(b) * a.num_heads + kvh * G + g) * D + lane * 8, q[g]);
        else
#pragma unroll
            for (int i = 0; i < 8; ++i) q[g][i] = 0.0f;
    }

    float m[GP], l[GP], acc[GP][8];
#pragma unroll
    for (int g = 0; g < GP; ++g)
    {
        m[g] = kNegBig;
        l[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
    }

    // U consecutive token groups per loop trip: their table entries, then all their K / V loads, go out before
    // any of them is used, so U times the bytes of one group are in flight per wave (fewer for fp32 caches, whose
    // raw rows take twice the registers, and none extra for the 16-head groups, which already fill them).
    constexpr int  U = GP >= 16 ? 1 : (Storage<CT>::bytes == 4 ? FFKV_GENERIC_U32 : FFKV_GENERIC_U16);
    // The table entries of the next trip are requested while this trip's tokens are computed.
    const int32_t* table = a.block_table + static_cast<int64_t>(b) * a.max_blocks;
    auto load_phys = [&](int base, int (&ph)[U])
    {
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            const int j = base + u * TPI + slot;
            ph[u] = j < end ? table[j >> 4] : -1;
        }
    };
    int phys[U];
    load_phys(begin, phys);
    for (int base = begin; base < end; base += U * TPI)
    {
        bool   valid[U];
        size_t row[U];
        float  ks[U], vs[U];  // int8: the tokens' scales
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            const int j = base + u * TPI + slot;
            valid[u] = j < end && phys[u] >= 0 && phys[u] < a.num_blocks;
            row[u] = (static_cast<size_t>(valid[u] ? phys[u] : 0) * kBlockSize + (j & 15)) * a.num_kv_heads + kvh;
        }
        Raw8 kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            ks[u] = vs[u] = 1.0f;
            if (valid[u] && act)
            {
                load_raw8<CT>(a.k_cache, row[u] * D + lane * 8, kr[u]);
                load_raw8<CT>(a.v_cache, row[u] * D + lane * 8, vr[u]);
                if constexpr (CT == I8)
                {
                    ks[u] = a.k_scale[row[u]];
                    vs[u] = a.v_scale[row[u]];
                }
            }
            else
            {
                kr[u] = Raw8{};
                vr[u] = Raw8{};
            }
        }
        load_phys(base + U * TPI, phys);
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            float k[8];
            unpack8<CT>(kr[u], k);
            if constexpr (CT == I8 || CT == FP8)
            {
                const float sk = CT == I8 ? ks[u] : a.k_scale[kvh];
#pragma unroll
                for (int i = 0; i < 8; ++i) k[i] *= sk;
            }
            float s[GP];
#pragma unroll
            for (int g = 0; g < GP; ++g)
            {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) d = __builtin_fmaf(q[g][i], k[i], d);
                s[g] = d;
            }
            // every lane takes part in the sums (DPP lane steps); a token's lanes are a contiguous, aligned group
#pragma unroll
            for (int g = 0; g < GP; ++g) s[g] = group_sum<LPT>(s[g]);

            // Online softmax with a lazy reference: m moves (and l, acc are rescaled) only when a score exceeds it
            // by more than 8 (log2 units), so p = 2^(s - m) < 2^8 and most tokens only add p and p * v.
            if (valid[u])
            {
                float v[8];  // unpacked only now: fewer registers live across the dot products and sums
                unpack8<CT>(vr[u], v);
                if constexpr (CT == I8 || CT == FP8)
                {
                    const float sv = CT == I8 ? vs[u] : a.v_scale[kvh];
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[i] *= sv;
                }
#pragma unroll
                for (int g = 0; g < GP; ++g)
                {
                    const float sg = s[g] * a.scale_log2;
                    if (sg > m[g] + 8.0f)
                    {
                        const float alpha = fast_exp2(m[g] - sg);  // 0 for the slot's first token
                        l[g] *= alpha;
#pragma unroll
                        for (int i = 0; i < 8; ++i) acc[g][i] *= alpha;
                        m[g] = sg;
                    }
                    const float p = fast_exp2(sg - m[g]);
                    l[g] += p;
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[g][i] = __builtin_fmaf(p, v[i], acc[g][i]);
                }
            }
        }
    }

    // merge the token slots of this wave (lanes lane, lane+LPT, ... hold the same dims)
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1)
    {
#pragma unroll
        for (int g = 0; g < GP; ++g)
        {
            const float mo = shfl_xor(m[g], off);
            const float lo = shfl_xor(l[g], off);
            const float mn = fmaxf(m[g], mo);
            const float a1 = fast_exp2(m[g] - mn);
            const float a2 = fast_exp2(mo - mn);
            l[g] = l[g] * a1 + lo * a2;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] = acc[g][i] * a1 + shfl_xor(acc[g][i], off) * a2;
            m[g] = mn;
        }
    }

    // merge the waves through LDS, one wave at a time
    __shared__ float s_acc[GP][DMAX];
    __shared__ float s_m[GP];
    __shared__ float s_l[GP];
    const bool holder = (tid % 64) < LPT && act;
    for (int w = 0; w < WAVES; ++w)
    {
        if (wave == w && holder)
        {
#pragma unroll
            for (int g = 0; g < GP; ++g)
            {
                if (w == 0)
                {
#pragma unroll
                    for (int i = 0; i < 8; ++i) s_acc[g][lane * 8 + i] = acc[g][i];
                    if (lane == 0)
                    {
                        s_m[g] = m[g];
                        s_l[g] = l[g];
                    }
                }
                else
                {
                    const float mo = s_m[g];
                    const float lo = s_l[g];
                    const float mn = fmaxf(m[g], mo);
                    const float a1 = fast_exp2(m[g] - mn);
                    const float a2 = fast_exp2(mo - mn);
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        s_acc[g][lane * 8 + i] = acc[g][i] * a1 + s_acc[g][lane * 8 + i] * a2;
                    // all holder lanes read s_m/s_l before lane 0 overwrites them: same wave, lockstep
                    __builtin_amdgcn_wave_barrier();
                    if (lane == 0)
                    {
                        s_m[g] = mn;
                        s_l[g] = l[g] * a1 + lo * a2;
                    }
                }
            }
        }
        __syncthreads();
    }

    const int     hq0 = kvh * G;
    const bool    single = nch <= 1;
    const int64_t ml_base = (static_cast<int64_t>(b) * a.num_heads + hq0) * a.max_chunks + chunk_id;
    for (int idx = tid; idx < G * D; idx += 256)
    {
        const int   g = idx / D;
        const int   d = idx % D;
        const float acc_v = s_acc[g][d];
        if (single)
        {
            const float lsum = s_l[g];
            store_act1(a.out, a.qo_dtype, (static_cast<size_t>(b) * a.num_heads + hq0 + g) * D + d,
                       lsum > 0.0f ? acc_v / lsum : 0.0f);
        }
        else
        {
            const int64_t pi = ml_base + static_cast<int64_t>(g) * a.max_chunks;
            a.ws_acc[pi * D + d] = acc_v;
            if (d == 0)
            {
                a.ws_ml[2 * pi] = s_m[g];
                a.ws_ml[2 * pi + 1] = s_l[g];
            }
        }
    }
}

// Combine the chunk partials of rows that needed more than one chunk.  One workgroup per (query head, row).
__global__ __launch_bounds__(256) void paged_decode_merge(DecodeArgs a)
{
    const int D = a.head_dim;
    const int hq = blockIdx.x;
    const int b = blockIdx.y;
    const int L = row_tokens(a, b);
    const int nch = (L + a.chunk - 1) / a.chunk;
    if (nch <= 1) return;

    const int64_t base = (static_cast<int64_t>(b) * a.num_heads + hq) * a.max_chunks;
    float         M = kNegBig;
    for (int c = 0; c < nch; ++c) M = fmaxf(M, a.ws_ml[2 * (base + c)]);
    float lsum = 0.0f;
    for (int c = 0; c < nch; ++c) lsum += a.ws_ml[2 * (base + c) + 1] * fast_exp2(a.ws_ml[2 * (base + c)] - M);
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    for (int d = threadIdx.x; d < D; d += 256)
    {
        float o = 0.0f;
        for (int c = 0; c < nch; ++c)
            o += a.ws_acc[(base + c) * D + d] * fast_exp2(a.ws_ml[2 * (base + c)] - M);
        store_act1(a.out, a.qo_dtype, (static_cast<size_t>(b) * a.num_heads + hq) * D + d, o * inv);
    }
}

namespace
{

template <int CT, int DT, int LPT, int GP>
hipError_t launch3(const DecodeArgs& a, hipStream_t stream)
{
    dim3 grid(static_cast<unsigned>(a.max_chunks), static_cast<unsigned>(a.num_kv_heads),
              static_cast<unsigned>(a.batch));
    hipLaunchKernelGGL((paged_decode_generic<CT, DT, LPT, GP>), grid, dim3(256), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.max_chunks <= 1) return e;
    hipLaunchKernelGGL(paged_decode_merge, dim3(static_cast<unsigned>(a.num_heads), static_cast<unsigned>(a.batch)),
                       dim3(a.head_dim < 256 ? a.head_dim : 256), 0, stream, a);
    return hipGetLastError();
}

template <int CT, int DT, int LPT>
hipError_t launch2(const DecodeArgs& a, hipStream_t stream)
{
    if (a.group <= 1) return launch3<CT, DT, LPT, 1>(a, stream);
    if (a.group <= 2) return launch3<CT, DT, LPT, 2>(a, stream);
    if (a.group <= 4) return launch3<CT, DT, LPT, 4>(a, stream);
    if (a.group <= 8) return launch3<CT, DT, LPT, 8>(a, stream);
    return launch3<CT, DT, LPT, 16>(a, stream);
}

template <int CT>
hipError_t launch1(const DecodeArgs& a, hipStream_t stream)
{
    switch (a.head_dim)
    {
        case 64:
            return launch2<CT, 64, 8>(a, stream);
        case 128:
            return launch2<CT, 128, 16>(a, stream);
        case 256:
            return launch2<CT, 256, 32>(a, stream);
        default:  // any other multiple of 8 up to 128: 16 lanes per token, those past head_dim / 8 idle
            return launch2<CT, 0, 16>(a, stream);
    }
}

}  // namespace

hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream)
{
    switch (a.cache_dtype)
    {
        case F32:
            return launch1<F32>(a, stream);
        case F16:
            return launch1<F16>(a, stream);
        case BF16:
            return launch1<BF16>(a, stream);
        case I8:
            return launch1<I8>(a, stream);
        default:
            return launch1<FP8>(a, stream);
    }
}

}  // namespace ffkv
