// paged_prefill.hip - chunked / paged prefill attention on gfx950 matrix cores.
//
// Replaces the reference's prefill branch of kernels::attention (flash_attn_wmma_kernel,
// src/kernels/attention.cu:22-286, dispatched at :460-474 and routed from src/model/qwen_model.cu:147-151), which
// attends only to the chunk's own contiguous K/V with a causal mask (key n > query m masked, :173-174) and so
// ignores any cached prefix.  Here query token t of row b sits at position ctx[b] + t and attends the keys
// 0 .. ctx[b] + t of the row read from the paged cache (prefix and chunk, after the chunk's append).  Without a
// block table the K/V are the chunk's contiguous [B, S, Hkv, D] tensors and ctx = 0: exactly the reference's
// causal prefill.  With S = 1 it is the decode attention.
//
// Mapping: a workgroup of eight waves serves 128 query rows of one (row b, kv head); a query row is a (token,
// head-in-group) pair, so GQA heads sharing a kv head share every K/V page.  Each wave owns 16 rows as the 16
// columns of its MFMA tiles, exactly as the decode kernel's columns are the heads of one kv head:
//   S^T[key, row] = K Q^T with K (16 keys x 32 dims) as the A operand from LDS and Q^T in registers,
//   online softmax per column (causal limit per column) over a step of pages at a time, O^T += V^T P^T as 16x16x32
//   products over those 32 keys with V^T read from a transposed LDS tile (8-byte reads) and P^T (split into two
//   16-bit parts) straight from the score registers.
// K/V pages are loaded once per workgroup by all its threads, four at a time (two at D = 256), converted to the
// MFMA type (8-bit codes too) and double-buffered in LDS: the next four pages are in flight while the current
// four are computed, one barrier per four pages.
#include "mfma_common.h"

namespace ffkv
{

#ifndef FFKV_PREFILL_WAVES
#define FFKV_PREFILL_WAVES 8  // waves per workgroup (16 query rows each)
#endif

#ifndef FFKV_PREFILL_KP
#define FFKV_PREFILL_KP 2  // pages per step at head_dim <= 128
#endif

#ifndef FFKV_PREFILL_DMA
#define FFKV_PREFILL_DMA 1  // 16-bit caches take paged_prefill_dma (global->LDS loads, transposed LDS reads)
#endif

#ifndef FFKV_PREFILL_DMA8
#define FFKV_PREFILL_DMA8 1  // so do int8 / fp8 caches (codes converted at operand-read time)
#endif
constexpr int kPfWaves = FFKV_PREFILL_WAVES;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = 16 * kPfWaves;  // query rows per workgroup

template <int CT, int QT, int D>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 4 : 1)))
void paged_prefill_mfma(PrefillArgs a)
{
    constexpr bool BF = kBF<CT, QT>;
    using M = MType<BF>;
    using X8 = typename M::x8;
    constexpr int  KSTEPS = D / 32;
    constexpr int  NT = D / 16;  // output tiles of 16 dims
    constexpr bool NEED_LO = !((QT == BF16 && BF) || (QT == F16 && !BF));
    constexpr bool Q8 = kElemBytes<CT> == 1;
    constexpr int  KP = D <= 128 ? FFKV_PREFILL_KP : 2;  // pages per step (one barrier per step), an even number
    constexpr int  RS = KP * kBlockSize + 4;    // row stride of the V^T tile (keys, padded against bank conflicts)
    constexpr int  CPT = D / 8;                 // 8-element chunks per key row
    constexpr int  CHUNKS = kBlockSize * CPT;   // chunks per page

    __shared__ uint16_t s_k[2][KP][kBlockSize * D];  // K rows (swizzled 16-byte chunks)
    __shared__ uint16_t s_vt[2][D * RS];             // V^T: dim-major, keys of the step's pages contiguous
    __shared__ float    s_ks[2][KP][kBlockSize];
    __shared__ float    s_vs[2][KP][kBlockSize];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int c = lane & 15;  // MFMA column = query row of this wave
    const int g = lane >> 4;  // lane group
    const int b = blockIdx.z;
    const int kvh = blockIdx.y;
    const int G = a.group;
    const int S = a.seq_len;
    const int Hq = a.num_heads;
    const int Hkv = a.num_kv_heads;
    const int R = S * G;  // query rows of (b, kvh)
    const int row0 = blockIdx.x * kPfRows;
    if (row0 >= R) return;  // uniform over the workgroup

    // keys of the row: L = ctx + S after the chunk's append (clamped); contiguous mode: the chunk only
    const int64_t ctx = a.paged ? static_cast<int64_t>(a.context_lens[b]) : 0;
    int64_t       Lr = ctx + S;
    if (a.paged && Lr > a.cap_tokens) Lr = a.cap_tokens;
    if (Lr < 0) Lr = 0;
    const int L = static_cast<int>(Lr);

    // this lane's query row: token t, head h; it sees keys [0, kend)
    const int  r = row0 + 16 * wave + c;
    const bool col_ok = r < R;
    const int  t = col_ok ? r / G : 0;
    const int  h = kvh * G + (col_ok ? r % G : 0);
    int64_t    ke = ctx + t + 1;
    ke = ke > L ? L : (ke < 0 ? 0 : ke);
    const int kend = col_ok ? static_cast<int>(ke) : 0;
    // pages the workgroup needs: up to its last query row's limit
    const int r_last = min(row0 + kPfRows, R) - 1;
    int64_t   kw = ctx + r_last / G + 1;
    kw = kw > L ? L : (kw < 0 ? 0 : kw);
    const int  pages = static_cast<int>((kw + kBlockSize - 1) / kBlockSize);
    const int  steps = (pages + KP - 1) / KP;
    const bool wave_active = row0 + 16 * wave < R;

    float kv_scale_log2 = a.scale_log2;
    float v_head_scale = 1.0f;
    if constexpr (CT == FP8)
    {
        kv_scale_log2 *= a.k_scale[kvh];
        v_head_scale = a.v_scale[kvh];
    }

    // ---- Q^T operands of the 16 query rows (column c), dims 32j + 8g .. +8 of k-step j --------------------------
    X8           qhi[KSTEPS], qlo[KSTEPS];
    const size_t qrow = (static_cast<size_t>(b) * S + t) * Hq + h;
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j)
    {
        const int d0 = 32 * j + 8 * g;
        if constexpr (!NEED_LO)
        {
            u32x4 w = u32x4{0u, 0u, 0u, 0u};
            if (col_ok) w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.q) + qrow * D + d0);
            qhi[j] = __builtin_bit_cast(X8, w);
            qlo[j] = qhi[j];
        }
        else
        {
            float x[8];
            if (col_ok)
                load_q8<QT>(a.q, qrow * D + d0, x);
            else
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = 0.0f;
            uint32_t hi[8], lo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
            {
                hi[e] = M::bits(x[e]);
                lo[e] = M::bits(x[e] - M::value(hi[e]));
            }
            qhi[j] = __builtin_bit_cast(X8, u32x4{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16), hi[4] | (hi[5] << 16),
                                                  hi[6] | (hi[7] << 16)});
            qlo[j] = __builtin_bit_cast(X8, u32x4{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16), lo[4] | (lo[5] << 16),
                                                  lo[6] | (lo[7] << 16)});
        }
    }

    // ---- cooperative loads of KP pages per step --------------------------------------------------------------
    // Block-table entries come 64 at a time (lane l of every wave: entry tb + l).
    int  tb = 0;
    auto load_tvec = [&](int base) -> int
    {
        return base + lane < a.max_blocks ? a.block_table[static_cast<int64_t>(b) * a.max_blocks + base + lane] : -1;
    };
    int tvec = a.paged ? load_tvec(0) : -1;

    // Each page is 2 * CHUNKS 16-byte units (K chunks, then V chunks); thread tid stages units tid, tid + threads,
    // ... of every page of a step, so with 8 waves at D = 128 waves 0-3 carry K and waves 4-7 carry V.
    constexpr int UNITS = 2 * CHUNKS;
    constexpr int PU = (UNITS + kPfThreads - 1) / kPfThreads;  // units per thread and page
    struct Stage
    {
        u32x4 w[KP][PU];       // 16-bit: 8 elements; 8-bit: codes in [0], [1]
        float ks[KP], vs[KP];  // int8 scales of key `tid` of each page (threads 0..15)
        bool  ok[KP];          // page present (and inside the row)
    };
    auto load_step = [&](int st_i, Stage& st)
    {
#pragma unroll
        for (int u = 0; u < KP; ++u)
        {
            const int pg = st_i * KP + u;
            int       phys = 0;
            bool      ok = pg < pages;
            if (ok && a.paged)
            {
                if (pg - tb >= 64)  // uniform
                {
                    tb += 64;
                    tvec = load_tvec(tb);
                }
                phys = __builtin_amdgcn_readlane(tvec, pg - tb);
                ok = phys >= 0 && phys < a.num_blocks;
            }
            st.ok[u] = ok;
#pragma unroll
            for (int i = 0; i < PU; ++i)
            {
                const int e = tid + kPfThreads * i;
                st.w[u][i] = u32x4{0u, 0u, 0u, 0u};
                if (!ok || e >= UNITS) continue;
                // K: chunk-major (consecutive threads read a token's row contiguously); V: token-major, so the
                // transposed LDS writes of consecutive threads land on consecutive keys of a V^T row
                const bool  is_k = e < CHUNKS;
                const int   f = is_k ? e : e - CHUNKS;
                const int   tok = is_k ? f / CPT : f % kBlockSize;
                const int   ch = is_k ? f % CPT : f / kBlockSize;
                const void* base = is_k ? a.k_cache : a.v_cache;
                if (pg * kBlockSize + tok >= L) continue;  // past the row's last key (contiguous: no such row)
                const size_t row = a.paged ? (static_cast<size_t>(phys) * kBlockSize + tok) * Hkv + kvh
                                           : (static_cast<size_t>(b) * S + pg * kBlockSize + tok) * Hkv + kvh;
                if constexpr (!Q8)
                {
                    st.w[u][i] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + row * D + 8 * ch);
                }
                else
                {
                    const u32x2 w8 = *reinterpret_cast<const u32x2*>(static_cast<const uint8_t*>(base) + row * D + 8 * ch);
                    st.w[u][i] = u32x4{w8[0], w8[1], 0u, 0u};
                }
            }
            if constexpr (CT == I8)
            {
                st.ks[u] = 0.0f;
                st.vs[u] = 0.0f;
                if (ok && tid < kBlockSize && pg * kBlockSize + tid < L)
                {
                    const size_t row = (static_cast<size_t>(phys) * kBlockSize + tid) * Hkv + kvh;
                    st.ks[u] = a.k_scale[row];
                    st.vs[u] = a.v_scale[row];
                }
            }
        }
    };
    auto store_step = [&](int buf, const Stage& st)
    {
#pragma unroll
        for (int u = 0; u < KP; ++u)
        {
#pragma unroll
            for (int i = 0; i < PU; ++i)
            {
                const int e = tid + kPfThreads * i;
                if (e >= UNITS) continue;
                const bool is_k = e < CHUNKS;
                const int  f = is_k ? e : e - CHUNKS;
                u32x4      w = st.w[u][i];
                if constexpr (Q8) w = codes_to_m<CT, BF>(st.w[u][i][0], st.w[u][i][1]);
                if (is_k)
                {
                    *reinterpret_cast<u32x4*>(&s_k[buf][u][lds_pos<D>(f / CPT, 8 * (f % CPT))]) = w;
                }
                else
                {
                    uint16_t* vt = &s_vt[buf][(8 * (f / kBlockSize)) * RS + u * kBlockSize + f % kBlockSize];
#pragma unroll
                    for (int e2 = 0; e2 < 8; ++e2) vt[e2 * RS] = static_cast<uint16_t>(w[e2 / 2] >> (16 * (e2 & 1)));
                }
            }
            if constexpr (CT == I8)
            {
                if (tid < kBlockSize)
                {
                    s_ks[buf][u][tid] = st.ks[u];
                    s_vs[buf][u][tid] = st.vs[u];
                }
            }
        }
    };

    // ---- per-wave flash step over one staged page -----------------------------------------------------------
    float m_run = kNegInf;  // running max of column c (log2 domain), equal in the four lane groups
    float l_run = 0.0f;     // this lane's share of the denominator (keys 4g..4g+3 of each page)
    f32x4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Pages u0 and u0 + 1 of a staged step.  The 32 keys form the k-slots of one 16x16x32 PV product: slot
    // 8g + e holds key 4g + e of page u0 for e < 4 and key 4g + e - 4 of page u0 + 1 otherwise, which is where the
    // two pages' score tiles leave them in lane (c, g); the V^T operand reads the same keys from the V^T tile.
    int kaddr[KSTEPS];  // K operand addresses (elements) within a page tile
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) kaddr[j] = lds_pos<D>(c, 32 * j + 8 * g);

    // One staged step of KP pages: the KP score tiles first (independent MFMA chains), one online-softmax update
    // over the step's 16 * KP keys, then the PV products page pair by page pair.
    auto compute_step = [&](int buf, int pg0, const bool* okp)
    {
        f32x4 s[KP];
#pragma unroll
        for (int u = 0; u < KP; ++u) s[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};  // lane (c, g): keys 4g + i, row c
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
#pragma unroll
            for (int u = 0; u < KP; ++u)
            {
                const X8 kj = __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(s_k[buf][u] + kaddr[j]));
                s[u] = M::mma32(kj, qhi[j], s[u]);
                if constexpr (NEED_LO) s[u] = M::mma32(kj, qlo[j], s[u]);
            }
        }
        float sc[KP * 4];
        float vs[KP * 4];
        float mt = kNegInf;
#pragma unroll
        for (int u = 0; u < KP; ++u)
        {
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                float ks = 1.0f;
                vs[4 * u + i] = 1.0f;
                if constexpr (CT == I8)
                {
                    ks = s_ks[buf][u][4 * g + i];
                    vs[4 * u + i] = s_vs[buf][u][4 * g + i];
                }
                const bool vis = okp[u] && (pg0 + u) * kBlockSize + 4 * g + i < kend;  // causal limit
                sc[4 * u + i] = vis ? s[u][i] * ks * kv_scale_log2 : kNegInf;
                mt = fmaxf(mt, sc[4 * u + i]);
            }
        }
        mt = xor_max(mt);
        const float m_new = fmaxf(m_run, mt);
        const float m_use = m_new == kNegInf ? 0.0f : m_new;  // a row with no visible key yet stays empty
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float       pv[KP * 4];
        float       psum = 0.0f;
#pragma unroll
        for (int e = 0; e < KP * 4; ++e)
        {
            const float pr = __builtin_amdgcn_exp2f(sc[e] - m_use);
            psum += pr;
            pv[e] = pr * vs[e];
        }
        l_run = l_run * alpha + psum;
        if (__any(m_new > m_run))
        {
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[n] *= alpha;
        }
        m_run = m_new;

        // Pages u0, u0 + 1 form the 32 k-slots of one 16x16x32 PV product: slot 8g + e holds key 4g + e of page
        // u0 for e < 4 and key 4g + e - 4 of page u0 + 1 otherwise, where the score tiles leave them in lane
        // (c, g); the V^T operand reads the same keys from the transposed tile.
        const uint16_t* vt = s_vt[buf] + c * RS + 4 * g;
#pragma unroll
        for (int u0 = 0; u0 < KP; u0 += 2)
        {
            uint32_t ph[8], pl[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
            {
                ph[e] = M::bits(pv[4 * u0 + e]);
                pl[e] = M::bits(pv[4 * u0 + e] - M::value(ph[e]));
            }
            const X8 phi = __builtin_bit_cast(X8, u32x4{ph[0] | (ph[1] << 16), ph[2] | (ph[3] << 16),
                                                        ph[4] | (ph[5] << 16), ph[6] | (ph[7] << 16)});
            const X8 plo = __builtin_bit_cast(X8, u32x4{pl[0] | (pl[1] << 16), pl[2] | (pl[3] << 16),
                                                        pl[4] | (pl[5] << 16), pl[6] | (pl[7] << 16)});
#pragma unroll
            for (int n = 0; n < NT; ++n)
            {
                const u32x2 a0 = *reinterpret_cast<const u32x2*>(vt + (16 * n) * RS + u0 * kBlockSize);
                const u32x2 a1 = *reinterpret_cast<const u32x2*>(vt + (16 * n) * RS + (u0 + 1) * kBlockSize);
                const X8    va = __builtin_bit_cast(X8, u32x4{a0[0], a0[1], a1[0], a1[1]});
                acc[n] = M::mma32(va, phi, acc[n]);
                acc[n] = M::mma32(va, plo, acc[n]);
            }
        }
    };

    // ---- steps of KP pages, double-buffered: step i + 1 in flight while step i is computed -------------------
    Stage st;
    bool  ok_cur[KP];
#pragma unroll
    for (int u = 0; u < KP; ++u) ok_cur[u] = false;
    if (steps > 0)
    {
        load_step(0, st);
        store_step(0, st);
#pragma unroll
        for (int u = 0; u < KP; ++u) ok_cur[u] = st.ok[u];
    }
    __syncthreads();
    for (int si = 0; si < steps; ++si)
    {
        const int buf = si & 1;
        bool      ok_next[KP];
#pragma unroll
        for (int u = 0; u < KP; ++u) ok_next[u] = false;
        if (si + 1 < steps)
        {
            load_step(si + 1, st);
#pragma unroll
            for (int u = 0; u < KP; ++u) ok_next[u] = st.ok[u];
        }
        bool any_ok = false;
#pragma unroll
        for (int u = 0; u < KP; ++u) any_ok = any_ok || ok_cur[u];
        if (wave_active && any_ok) compute_step(buf, si * KP, ok_cur);
        if (si + 1 < steps) store_step(buf ^ 1, st);  // that buffer was last read before the previous barrier
        __syncthreads();
#pragma unroll
        for (int u = 0; u < KP; ++u) ok_cur[u] = ok_next[u];
    }

    if (col_ok)
    {
        const float l_tot = xor_sum(l_run);
        const float inv = l_tot > 0.0f ? v_head_scale / l_tot : 0.0f;
        const size_t ob = qrow * D;
#pragma unroll
        for (int n = 0; n < NT; ++n) store_out4<QT>(a.out, ob + 16 * n + 4 * g, acc[n] * inv);
    }
}

namespace
{

template <int CT, int QT>
hipError_t launch_pf_d(const PrefillArgs& a, hipStream_t stream)
{
    const int  rows = a.seq_len * a.group;
    const dim3 grid(static_cast<unsigned>((rows + kPfRows - 1) / kPfRows), static_cast<unsigned>(a.num_kv_heads),
                    static_cast<unsigned>(a.batch));
    switch (a.head_dim)
    {
        case 64:
            hipLaunchKernelGGL((paged_prefill_mfma<CT, QT, 64>), grid, dim3(kPfThreads), 0, stream, a);
            break;
        case 128:
            hipLaunchKernelGGL((paged_prefill_mfma<CT, QT, 128>), grid, dim3(kPfThreads), 0, stream, a);
            break;
        default:
            hipLaunchKernelGGL((paged_prefill_mfma<CT, QT, 256>), grid, dim3(kPfThreads), 0, stream, a);
            break;
    }
    return hipGetLastError();
}

template <int CT>
hipError_t launch_pf_q(const PrefillArgs& a, hipStream_t stream)
{
    switch (a.qo_dtype)
    {
        case F32:
            return launch_pf_d<CT, F32>(a, stream);
        case F16:
            return launch_pf_d<CT, F16>(a, stream);
        default:
            return launch_pf_d<CT, BF16>(a, stream);
    }
}

}  // namespace

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream)
{
#if FFKV_PREFILL_DMA
    if (a.cache_dtype == F16 || a.cache_dtype == BF16 || FFKV_PREFILL_DMA8) return launch_prefill_dma(a, stream);
#endif
    switch (a.cache_dtype)
    {
        case F16:
            return launch_pf_q<F16>(a, stream);
        case BF16:
            return launch_pf_q<BF16>(a, stream);
        case I8:
            return launch_pf_q<I8>(a, stream);
        default:
            return launch_pf_q<FP8>(a, stream);
    }
}

}  // namespace ffkv
