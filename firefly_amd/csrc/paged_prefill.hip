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
// Mapping: a workgroup of four waves serves 64 query rows of one (row b, kv head); a query row is a (token,
// head-in-group) pair, so GQA heads sharing a kv head share every K/V page.  Each wave owns 16 rows as the 16
// columns of its MFMA tiles, exactly as the decode kernel's columns are the heads of one kv head:
//   S^T[key, row] = K Q^T with K (16 keys x 32 dims) as the A operand from LDS and Q^T in registers,
//   online softmax per column (causal limit per column), O^T += V^T P^T with V^T read from LDS and P^T (split
//   into two 16-bit parts) straight from the score registers.
// K/V pages are loaded once per workgroup by all 256 threads, converted to the MFMA type (8-bit codes too) and
// double-buffered in LDS: page p + 1 is in flight while page p is computed, one barrier per page.
#include "mfma_common.h"

namespace ffkv
{

template <int CT, int QT, int D>
__global__ __launch_bounds__(256) void paged_prefill_mfma(PrefillArgs a)
{
    constexpr bool BF = kBF<CT, QT>;
    using M = MType<BF>;
    using X8 = typename M::x8;
    constexpr int  KSTEPS = D / 32;
    constexpr int  NT = D / 16;  // output tiles of 16 dims
    constexpr bool NEED_LO = !((QT == BF16 && BF) || (QT == F16 && !BF));
    constexpr bool Q8 = kElemBytes<CT> == 1;
    constexpr int  CPT = D / 8;                 // 8-element chunks per key row
    constexpr int  CHUNKS = kBlockSize * CPT;   // chunks per page
    constexpr int  PER = (CHUNKS + 255) / 256;  // chunks per thread

    __shared__ uint16_t s_k[2][kBlockSize * D];
    __shared__ uint16_t s_v[2][kBlockSize * D];
    __shared__ float    s_ks[2][kBlockSize];
    __shared__ float    s_vs[2][kBlockSize];

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
    const int row0 = blockIdx.x * 64;
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
    const int r_last = min(row0 + 64, R) - 1;
    int64_t   kw = ctx + r_last / G + 1;
    kw = kw > L ? L : (kw < 0 ? 0 : kw);
    const int  pages = static_cast<int>((kw + kBlockSize - 1) / kBlockSize);
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

    // ---- cooperative page loads ----------------------------------------------------------------------------
    // Block-table entries come 64 at a time (lane l of every wave: entry tb + l).
    int  tb = 0;
    auto load_tvec = [&](int base) -> int
    {
        return base + lane < a.max_blocks ? a.block_table[static_cast<int64_t>(b) * a.max_blocks + base + lane] : -1;
    };
    int tvec = a.paged ? load_tvec(0) : -1;

    struct Stage
    {
        u32x4 k[PER];  // 16-bit: 8 elements; 8-bit: codes in .x, .y
        u32x4 v[PER];
        float ks, vs;  // int8 scales of key `tid` (threads 0..15)
        bool  ok;      // page present
    };
    auto load_page = [&](int pg, Stage& st)
    {
        int  phys = 0;
        bool ok = true;
        if (a.paged)
        {
            if (pg - tb >= 64)  // uniform
            {
                tb += 64;
                tvec = load_tvec(tb);
            }
            phys = __builtin_amdgcn_readlane(tvec, pg - tb);
            ok = phys >= 0 && phys < a.num_blocks;
        }
        st.ok = ok;
        if (!ok) return;
#pragma unroll
        for (int i = 0; i < PER; ++i)
        {
            const int e = tid + 256 * i;
            st.k[i] = u32x4{0u, 0u, 0u, 0u};
            st.v[i] = u32x4{0u, 0u, 0u, 0u};
            if (e >= CHUNKS) continue;
            const int tok = e / CPT, ch = e % CPT;
            if (pg * kBlockSize + tok >= L) continue;  // past the row's last key (contiguous: no such row)
            const size_t row = a.paged ? (static_cast<size_t>(phys) * kBlockSize + tok) * Hkv + kvh
                                       : (static_cast<size_t>(b) * S + pg * kBlockSize + tok) * Hkv + kvh;
            if constexpr (!Q8)
            {
                st.k[i] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.k_cache) + row * D + 8 * ch);
                st.v[i] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.v_cache) + row * D + 8 * ch);
            }
            else
            {
                const u32x2 kw8 = *reinterpret_cast<const u32x2*>(static_cast<const uint8_t*>(a.k_cache) + row * D + 8 * ch);
                const u32x2 vw8 = *reinterpret_cast<const u32x2*>(static_cast<const uint8_t*>(a.v_cache) + row * D + 8 * ch);
                st.k[i] = u32x4{kw8[0], kw8[1], 0u, 0u};
                st.v[i] = u32x4{vw8[0], vw8[1], 0u, 0u};
            }
        }
        if constexpr (CT == I8)
        {
            st.ks = 0.0f;
            st.vs = 0.0f;
            if (tid < kBlockSize && pg * kBlockSize + tid < L)
            {
                const size_t row = (static_cast<size_t>(phys) * kBlockSize + tid) * Hkv + kvh;
                st.ks = a.k_scale[row];
                st.vs = a.v_scale[row];
            }
        }
    };
    auto store_page = [&](int buf, const Stage& st)
    {
#pragma unroll
        for (int i = 0; i < PER; ++i)
        {
            const int e = tid + 256 * i;
            if (e >= CHUNKS) continue;
            const int tok = e / CPT, ch = e % CPT;
            u32x4     kw = u32x4{0u, 0u, 0u, 0u}, vw = u32x4{0u, 0u, 0u, 0u};
            if (st.ok)
            {
                if constexpr (!Q8)
                {
                    kw = st.k[i];
                    vw = st.v[i];
                }
                else
                {
                    kw = codes_to_m<CT, BF>(st.k[i][0], st.k[i][1]);
                    vw = codes_to_m<CT, BF>(st.v[i][0], st.v[i][1]);
                }
            }
            *reinterpret_cast<u32x4*>(&s_k[buf][lds_pos<D>(tok, 8 * ch)]) = kw;
            *reinterpret_cast<u32x4*>(&s_v[buf][lds_pos<D>(tok, 8 * ch)]) = vw;
        }
        if constexpr (CT == I8)
        {
            if (tid < kBlockSize)
            {
                s_ks[buf][tid] = st.ok ? st.ks : 0.0f;
                s_vs[buf][tid] = st.ok ? st.vs : 0.0f;
            }
        }
    };

    // ---- per-wave flash step over one staged page -----------------------------------------------------------
    float m_run = kNegInf;  // running max of column c (log2 domain), equal in the four lane groups
    float l_run = 0.0f;     // this lane's share of the denominator (keys 4g..4g+3 of each page)
    f32x4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int buf, int pg)
    {
        const uint16_t* sk = s_k[buf];
        const uint16_t* sv = s_v[buf];
        f32x4           s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};  // lane (c, g): keys 4g + i of query row c
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
            const X8 kj = __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(sk + lds_pos<D>(c, 32 * j + 8 * g)));
            s = M::mma32(kj, qhi[j], s);
            if constexpr (NEED_LO) s = M::mma32(kj, qlo[j], s);
        }
        float ks[4], vs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            ks[i] = 1.0f;
            vs[i] = 1.0f;
            if constexpr (CT == I8)
            {
                ks[i] = s_ks[buf][4 * g + i];
                vs[i] = s_vs[buf][4 * g + i];
            }
        }
        float sc[4];
        float mt = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const bool vis = pg * kBlockSize + 4 * g + i < kend;  // causal limit of this query row
            sc[i] = vis ? s[i] * ks[i] * kv_scale_log2 : kNegInf;
            mt = fmaxf(mt, sc[i]);
        }
        mt = xor_max(mt);
        const float m_new = fmaxf(m_run, mt);
        const float m_use = m_new == kNegInf ? 0.0f : m_new;  // a row with no visible key yet stays empty
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float       pv[4];
        float       psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const float pr = __builtin_amdgcn_exp2f(sc[i] - m_use);
            psum += pr;
            pv[i] = pr * vs[i];
        }
        l_run = l_run * alpha + psum;
        if (__any(m_new > m_run))
        {
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[n] *= alpha;
        }
        m_run = m_new;

        uint32_t ph[4], pl[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            ph[i] = M::bits(pv[i]);
            pl[i] = M::bits(pv[i] - M::value(ph[i]));
        }
        const typename M::x4 phi =
            __builtin_bit_cast(typename M::x4, u32x2{ph[0] | (ph[1] << 16), ph[2] | (ph[3] << 16)});
        const typename M::x4 plo =
            __builtin_bit_cast(typename M::x4, u32x2{pl[0] | (pl[1] << 16), pl[2] | (pl[3] << 16)});
#pragma unroll
        for (int n = 0; n < NT; ++n)
        {
            const uint32_t v0 = sv[lds_pos<D>(4 * g + 0, 16 * n + c)];
            const uint32_t v1 = sv[lds_pos<D>(4 * g + 1, 16 * n + c)];
            const uint32_t v2 = sv[lds_pos<D>(4 * g + 2, 16 * n + c)];
            const uint32_t v3 = sv[lds_pos<D>(4 * g + 3, 16 * n + c)];
            const typename M::x4 vt = __builtin_bit_cast(typename M::x4, u32x2{v0 | (v1 << 16), v2 | (v3 << 16)});
            acc[n] = M::mma16(vt, phi, acc[n]);
            acc[n] = M::mma16(vt, plo, acc[n]);
        }
    };

    // ---- pages 0 .. pages-1, double-buffered -----------------------------------------------------------------
    Stage st;
    bool  ok_cur = false;
    if (pages > 0)
    {
        load_page(0, st);
        store_page(0, st);
        ok_cur = st.ok;
    }
    __syncthreads();
    for (int pg = 0; pg < pages; ++pg)
    {
        const int buf = pg & 1;
        bool      ok_next = false;
        if (pg + 1 < pages)
        {
            load_page(pg + 1, st);  // in flight while page pg is computed
            ok_next = st.ok;
        }
        if (wave_active && ok_cur) compute(buf, pg);
        if (pg + 1 < pages) store_page(buf ^ 1, st);  // that buffer was last read before the previous barrier
        __syncthreads();
        ok_cur = ok_next;
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
    const dim3 grid(static_cast<unsigned>((rows + 63) / 64), static_cast<unsigned>(a.num_kv_heads),
                    static_cast<unsigned>(a.batch));
    switch (a.head_dim)
    {
        case 64:
            hipLaunchKernelGGL((paged_prefill_mfma<CT, QT, 64>), grid, dim3(256), 0, stream, a);
            break;
        case 128:
            hipLaunchKernelGGL((paged_prefill_mfma<CT, QT, 128>), grid, dim3(256), 0, stream, a);
            break;
        default:
            hipLaunchKernelGGL((paged_prefill_mfma<CT, QT, 256>), grid, dim3(256), 0, stream, a);
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
