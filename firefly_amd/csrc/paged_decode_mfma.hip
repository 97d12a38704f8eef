// paged_decode_mfma.hip - PagedAttention decode on the gfx950 matrix cores, split evenly over pages.
//
// Reference semantics: paged_attention_kernel (src/kernels/attention.cu:291-447): out[b, h] = softmax over the
// context_lens[b] + 1 cached tokens of scale * q[b, h] . k_j, applied to v_j, with kv_head = h / (Hq / Hkv).
//
// Design (one wave = one KV head of one page range; a page = 16 tokens = one MFMA tile):
//   * QK^T on MFMA: S^T[t, h] = K[t, :] . Q[h, :] with v_mfma_f32_16x16x32_{bf16,f16}; the 16 tokens of a page
//     are the rows, the (up to 16) query heads of the GQA group the columns.  K is fed straight from its page:
//     lane (c, g) = (lane % 16, lane / 16) loads token c's 16-byte run at dim 32j + 8g for k-step j, so one load
//     instruction covers 64 contiguous bytes of each of the 16 tokens.  The reduction over head_dim happens in
//     the matrix core; no cross-lane dot-product trees.
//   * softmax in base 2 (log2 e folded into the scale) on the MFMA output layout: lane (c, g) holds head c for
//     tokens 4g..4g+3, so the per-page max is 3 in-lane maxes and two cross-lane steps; the denominator stays a
//     per-lane partial sum until the end.
//   * PV on MFMA: O^T[d, h] += V^T[d, t] P^T[t, h] with v_mfma_f32_16x16x16; P^T is exactly the QK output
//     layout (k = token = 4g + i), V^T comes from an LDS copy of the page's V rows whose 32-byte chunks are
//     XOR-swizzled by token / 4, so the four token rows a read instruction touches fall in distinct bank
//     groups while every row stays 16-byte aligned for the vector writes.
//     P is split into hi + lo parts of the MFMA input type, so the products carry ~16 significant bits.
//   * quantized caches: int8 and fp8 e4m3 codes convert exactly to f16 for the MFMA; int8 per-token K scales
//     multiply the scores and V scales multiply P, fp8 per-head scales fold into the score scale and the output.
//   * work split: the pages of all rows form one sequence; work item i of W takes pages
//     [i*P/W, (i+1)*P/W), so every wave gets the same number of pages whatever the row lengths (no tail of
//     long rows).  A row covered by one item writes its output directly; otherwise each piece writes an
//     unnormalised partial (m, l, acc) to slot item + row and paged_decode_merge combines them.
#include "ffkv_device.h"
#include "ffkv_internal.h"

namespace ffkv
{

namespace
{

using f32x4 = float __attribute__((ext_vector_type(4)));
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using bf16x4 = __bf16 __attribute__((ext_vector_type(4)));
using f16x8 = _Float16 __attribute__((ext_vector_type(8)));
using f16x4 = _Float16 __attribute__((ext_vector_type(4)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));

constexpr float kNegInf = -__builtin_huge_valf();

// MFMA input element type: bf16 for bf16 caches, f16 for f16, int8 and fp8 caches (codes of both quantized
// formats are exact in f16).
template <bool BF>
struct MType;
template <>
struct MType<true>
{
    using x8 = bf16x8;
    using x4 = bf16x4;
    static __device__ __forceinline__ uint32_t bits(float x) { return f32_to_bf16(x); }
    static __device__ __forceinline__ float value(uint32_t h) { return bf16_to_f32(h); }
    static __device__ __forceinline__ f32x4 mma32(x8 a, x8 b, f32x4 c)
    {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 mma16(x4 a, x4 b, f32x4 c)
    {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    }
};
template <>
struct MType<false>
{
    using x8 = f16x8;
    using x4 = f16x4;
    static __device__ __forceinline__ uint32_t bits(float x)
    {
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    }
    static __device__ __forceinline__ float value(uint32_t h) { return f16_to_f32(h); }
    static __device__ __forceinline__ f32x4 mma32(x8 a, x8 b, f32x4 c)
    {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 mma16(x4 a, x4 b, f32x4 c)
    {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
};

template <int CT>
constexpr bool kBF = CT == BF16;
template <int CT>
constexpr int kElemBytes = (CT == I8 || CT == FP8) ? 1 : 2;

// First of the 8 dims that k-step j gives to lane group g.  Any bijection works as long as Q and K use the same
// one; these make each load instruction read contiguous bytes of every token (16-bit: 64 B, 8-bit: 16-byte
// loads that span two k-steps).
template <int CT>
__device__ __forceinline__ int dim_of(int j, int g)
{
    if constexpr (kElemBytes<CT> == 2)
        return 32 * j + 8 * g;
    else
        return 64 * (j >> 1) + 16 * g + 8 * (j & 1);
}

// 8 cache codes (one k-step of one lane) as 4 packed 16-bit MFMA words.  Quantized codes convert exactly.
template <int CT>
__device__ __forceinline__ u32x4 codes_to_m(uint32_t lo, uint32_t hi)
{
    uint32_t w[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
    {
        const uint32_t byte = ((e < 4 ? lo : hi) >> (8 * (e & 3))) & 0xffu;
        float          x;
        if constexpr (CT == I8)
            x = static_cast<float>(static_cast<int8_t>(byte));
        else
            x = e4m3_to_f32(byte);
        w[e] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    }
    return u32x4{w[0] | (w[1] << 16), w[2] | (w[3] << 16), w[4] | (w[5] << 16), w[6] | (w[7] << 16)};
}

template <int QT>
__device__ __forceinline__ void load_q8(const void* q, size_t i, float* x)
{
    Raw8 r;
    load_raw8<QT>(q, i, r);
    unpack8<QT>(r, x);
}

template <int QT>
__device__ __forceinline__ void store_out4(void* out, size_t i, f32x4 v)
{
    if constexpr (QT == F32)
    {
        *reinterpret_cast<f32x4*>(static_cast<float*>(out) + i) = v;
    }
    else
    {
        uint32_t h[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) h[k] = QT == BF16 ? f32_to_bf16(v[k]) : f32_to_f16(v[k]);
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + i) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
}

__device__ __forceinline__ int row_pages(const DecodeArgs& a, int b)
{
    int64_t L = static_cast<int64_t>(a.context_lens[b]) + 1;  // +1: the token appended this step (:320)
    if (L > a.cap_tokens) L = a.cap_tokens;
    if (L < 0) L = 0;
    return static_cast<int>((L + kBlockSize - 1) / kBlockSize);
}

__device__ __forceinline__ int row_tokens(const DecodeArgs& a, int b)
{
    int64_t L = static_cast<int64_t>(a.context_lens[b]) + 1;
    if (L > a.cap_tokens) L = a.cap_tokens;
    return L < 0 ? 0 : static_cast<int>(L);
}

// Position (16-bit elements) of V[t][d] in a wave's LDS tile of 16 rows x D: chunk d/16 of row t is stored at
// chunk (d/16) ^ ((t/4) % 4).
template <int D>
__device__ __forceinline__ int lds_pos(int t, int d)
{
    return t * D + ((((d >> 4) ^ ((t >> 2) & 3))) << 4) + (d & 15);
}

__device__ __forceinline__ float xor_max(float x)
{
    x = fmaxf(x, __shfl_xor(x, 16, 64));
    return fmaxf(x, __shfl_xor(x, 32, 64));
}

__device__ __forceinline__ float xor_sum(float x)
{
    x += __shfl_xor(x, 16, 64);
    return x + __shfl_xor(x, 32, 64);
}

}  // namespace

// Waves per SIMD the register budget is sized for: 4 (128 registers) where that fits without spills.
template <int CT, int QT, int D>
constexpr int kMfmaWaves =
    D == 256 ? 2 : ((D == 128 && !((QT == BF16 && CT == BF16) || (QT == F16 && CT == F16))) ? 3 : 4);

// Work item i (blockIdx.x) of W (gridDim.x); KV heads blockIdx.y*NW .. +NW, one per wave.
template <int CT, int QT, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kMfmaWaves<CT, QT, D>, 8))) void
paged_decode_mfma(DecodeArgs a)
{
    constexpr bool BF = kBF<CT>;
    using M = MType<BF>;
    constexpr int  KSTEPS = D / 32;
    constexpr int  NT = D / 16;                          // output tiles of 16 dims
    constexpr bool NEED_LO = !((QT == BF16 && BF) || (QT == F16 && !BF));

    __shared__ uint16_t s_v[4][kBlockSize * D];
    __shared__ int64_t  s_scan[4];
    __shared__ int64_t  s_total;
    __shared__ int      s_b0;
    __shared__ int64_t  s_pb0;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int c = lane & 15;  // MFMA column / row-in-tile index
    const int g = lane >> 4;  // lane group
    const int nthreads = blockDim.x;
    const int B = a.batch;

    // ---- pages per row, block-wide exclusive scan (each thread owns a contiguous run of rows) ------------
    const int per = (B + nthreads - 1) / nthreads;
    const int r0 = min(B, tid * per);
    const int r1 = min(B, r0 + per);
    int64_t   local = 0;
    for (int r = r0; r < r1; ++r) local += row_pages(a, r);
    int64_t incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
    {
        const int64_t o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
    }
    if (lane == 63) s_scan[wave] = incl;
    __syncthreads();
    int64_t wave_base = 0;
    for (int w = 0; w < wave; ++w) wave_base += s_scan[w];
    if (tid == nthreads - 1) s_total = wave_base + incl;
    __syncthreads();
    const int64_t P = s_total;
    const int64_t W = min(static_cast<int64_t>(gridDim.x), P);
    const int64_t item = blockIdx.x;
    if (item >= W) return;  // uniform over the workgroup; no barrier follows for returned threads' waves
    const int64_t start = item * P / W;
    const int64_t end = (item + 1) * P / W;
    const int64_t excl = wave_base + incl - local;
    if (excl <= start && start < excl + local)
    {
        int64_t pb = excl;
        int     r = r0;
        for (;; ++r)
        {
            const int n = row_pages(a, r);
            if (start < pb + n) break;
            pb += n;
        }
        s_b0 = r;
        s_pb0 = pb;
    }
    __syncthreads();

    const int kvh = blockIdx.y * (nthreads >> 6) + wave;
    if (kvh >= a.num_kv_heads) return;
    const int G = a.group;
    uint16_t* sv = s_v[wave];

    float kv_scale_log2 = a.scale_log2;
    float v_head_scale = 1.0f;
    if constexpr (CT == FP8)
    {
        kv_scale_log2 *= a.k_scale[kvh];
        v_head_scale = a.v_scale[kvh];
    }

    int     b = s_b0;
    int64_t pb = s_pb0;
    int     nb = row_pages(a, b);
    int64_t p = start;
    while (p < end)
    {
        const int64_t seg_end = min(end, pb + nb);
        const int     Lp = row_tokens(a, b);

        // ---- Q of this row's group as MFMA B operands (column c = head, zero beyond the group) ----------
        typename M::x8 qhi[KSTEPS], qlo[KSTEPS];
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
            float x[8];
            if (c < G)
                load_q8<QT>(a.q, (static_cast<size_t>(b) * a.num_heads + kvh * G + c) * D + dim_of<CT>(j, g), x);
            else
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = 0.0f;
            uint32_t hi[8], lo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
            {
                hi[e] = M::bits(x[e]);
                lo[e] = NEED_LO ? M::bits(x[e] - M::value(hi[e])) : 0u;
            }
            qhi[j] = __builtin_bit_cast(typename M::x8, u32x4{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16),
                                                             hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16)});
            qlo[j] = __builtin_bit_cast(typename M::x8, u32x4{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16),
                                                             lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16)});
        }

        float m_run = kNegInf;  // running max of head c (log2 domain), equal in the four lane groups
        float l_run = 0.0f;     // this lane's share of the denominator (tokens 4g..4g+3 of each page)
        f32x4 acc[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

        const int32_t* table = a.block_table + static_cast<int64_t>(b) * a.max_blocks;
        for (int pg = static_cast<int>(p - pb); pg < static_cast<int>(seg_end - pb); ++pg)
        {
            const int phys = table[pg];
            if (phys < 0 || phys >= a.num_blocks) continue;  // uniform: masked page
            const int n_tok = min(kBlockSize, Lp - pg * kBlockSize);

            // ---- load K (A operand rows = tokens) and V (to LDS) of token c ----------------------------
            const size_t row_c = (static_cast<size_t>(phys) * kBlockSize + c) * a.num_kv_heads + kvh;
            const bool   tok_ok = c < n_tok;
            typename M::x8 kop[KSTEPS];
            u32x4          vraw[KSTEPS];
            if constexpr (kElemBytes<CT> == 2)
            {
                const char* kp = static_cast<const char*>(a.k_cache) + row_c * D * 2;
                const char* vp = static_cast<const char*>(a.v_cache) + row_c * D * 2;
#pragma unroll
                for (int j = 0; j < KSTEPS; ++j)
                {
                    kop[j] = __builtin_bit_cast(typename M::x8,
                                                *reinterpret_cast<const u32x4*>(kp + dim_of<CT>(j, g) * 2));
                    vraw[j] = *reinterpret_cast<const u32x4*>(vp + dim_of<CT>(j, g) * 2);
                }
            }
            else
            {
                const char* kp = static_cast<const char*>(a.k_cache) + row_c * D;
                const char* vp = static_cast<const char*>(a.v_cache) + row_c * D;
#pragma unroll
                for (int j = 0; j < KSTEPS; j += 2)
                {
                    const u32x4 kw = *reinterpret_cast<const u32x4*>(kp + dim_of<CT>(j, g));
                    const u32x4 vw = *reinterpret_cast<const u32x4*>(vp + dim_of<CT>(j, g));
                    kop[j] = __builtin_bit_cast(typename M::x8, codes_to_m<CT>(kw[0], kw[1]));
                    kop[j + 1] = __builtin_bit_cast(typename M::x8, codes_to_m<CT>(kw[2], kw[3]));
                    vraw[j] = codes_to_m<CT>(vw[0], vw[1]);
                    vraw[j + 1] = codes_to_m<CT>(vw[2], vw[3]);
                }
            }
            // stage V[t = c] (zero for slots past the row's last token) into the wave's LDS tile
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j)
            {
                const u32x4 w = tok_ok ? vraw[j] : u32x4{0u, 0u, 0u, 0u};
                *reinterpret_cast<u32x4*>(sv + lds_pos<D>(c, dim_of<CT>(j, g))) = w;
            }

            // ---- S^T = K Q^T: lane (c, g) gets tokens 4g + i of head c ----------------------------------
            f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j)
            {
                s = M::mma32(kop[j], qhi[j], s);
                if constexpr (NEED_LO) s = M::mma32(kop[j], qlo[j], s);
            }

            float ks[4], vs[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                ks[i] = 1.0f;
                vs[i] = 1.0f;
            }
            if constexpr (CT == I8)
            {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    const size_t srow = (static_cast<size_t>(phys) * kBlockSize + 4 * g + i) * a.num_kv_heads + kvh;
                    ks[i] = a.k_scale[srow];
                    vs[i] = a.v_scale[srow];
                }
            }
            float sc[4];
            float mt = kNegInf;
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const bool ok = 4 * g + i < n_tok;
                sc[i] = ok ? s[i] * ks[i] * kv_scale_log2 : kNegInf;
                mt = fmaxf(mt, sc[i]);
            }
            mt = xor_max(mt);
            const float m_new = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            float       pv[4];
            float       psum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const float pr = __builtin_amdgcn_exp2f(sc[i] - m_new);
                psum += pr;
                pv[i] = 4 * g + i < n_tok ? pr * vs[i] : 0.0f;
            }
            l_run = l_run * alpha + psum;
            if (__any(m_new > m_run))
            {
#pragma unroll
                for (int n = 0; n < NT; ++n) acc[n] *= alpha;
            }
            m_run = m_new;

            // P^T as MFMA B operands (k = token 4g + i, column c = head), hi + lo parts
            uint32_t ph[4], pl[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                ph[i] = M::bits(pv[i]);
                pl[i] = M::bits(pv[i] - M::value(ph[i]));
            }
            const typename M::x4 phi = __builtin_bit_cast(typename M::x4, u32x2{ph[0] | (ph[1] << 16), ph[2] | (ph[3] << 16)});
            const typename M::x4 plo = __builtin_bit_cast(typename M::x4, u32x2{pl[0] | (pl[1] << 16), pl[2] | (pl[3] << 16)});

            // LDS writes of this wave are complete before its reads below (in-order LDS queue of one wave);
            // the fence keeps the compiler from moving the reads above the writes.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

            // ---- O^T[d, h] += V^T[d, t] P^T[t, h] over the 16 dims of each tile -------------------------
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
            // the next page's LDS writes must not overtake these reads
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }

        // ---- finish the row segment ---------------------------------------------------------------------
        const float l_tot = xor_sum(l_run);
        const int   h = kvh * G + c;
        const bool  whole = p == pb && seg_end == pb + nb;
        if (whole)
        {
            if (c < G)
            {
                const float inv = l_tot > 0.0f ? v_head_scale / l_tot : 0.0f;
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    store_out4<QT>(a.out, (static_cast<size_t>(b) * a.num_heads + h) * D + 16 * n + 4 * g,
                                   acc[n] * inv);
            }
        }
        else
        {
            const int64_t slot = item + b;
            if (c < G)
            {
                float* dst = a.ws_acc + (slot * a.num_heads + h) * D;
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    *reinterpret_cast<f32x4*>(dst + 16 * n + 4 * g) = acc[n] * v_head_scale;
                if (g == 0)
                {
                    a.ws_ml[(slot * a.num_heads + h) * 2] = m_run;
                    a.ws_ml[(slot * a.num_heads + h) * 2 + 1] = l_tot;
                }
            }
        }
        // the item holding a row's first page records which items cover the row
        if (p == pb && blockIdx.y == 0 && wave == 0 && lane == 0)
        {
            const int64_t last = pb + nb - 1;
            const int64_t i_hi = ((last + 1) * W + P - 1) / P - 1;  // largest i with i*P/W <= last
            a.ws_meta[2 * b] = static_cast<int32_t>(item);
            a.ws_meta[2 * b + 1] = static_cast<int32_t>(i_hi);
        }

        p = seg_end;
        if (p < end)
        {
            pb += nb;
            ++b;
            nb = row_pages(a, b);
            while (nb == 0)
            {
                ++b;
                nb = row_pages(a, b);
            }
        }
    }
}

// Combine the partials of rows split over several work items; write zeros for rows without tokens.
// One workgroup per (row, 256 / D heads).
template <int QT, int D>
__global__ __launch_bounds__(256) void paged_decode_mfma_merge(DecodeArgs a)
{
    constexpr int HPW = 256 / D;
    const int     b = blockIdx.x;
    const int     h = blockIdx.y * HPW + threadIdx.x / D;
    const int     d = threadIdx.x % D;
    if (h >= a.num_heads) return;
    const size_t oi = (static_cast<size_t>(b) * a.num_heads + h) * D + d;
    if (row_pages(a, b) == 0)
    {
        store_act1(a.out, QT, oi, 0.0f);
        return;
    }
    const int i_lo = a.ws_meta[2 * b];
    const int i_hi = a.ws_meta[2 * b + 1];
    if (i_lo == i_hi) return;  // written by the decode kernel
    float M = kNegInf;
    for (int i = i_lo; i <= i_hi; ++i) M = fmaxf(M, a.ws_ml[((static_cast<int64_t>(i) + b) * a.num_heads + h) * 2]);
    float o = 0.0f, lsum = 0.0f;
    if (M != kNegInf)
    {
        for (int i = i_lo; i <= i_hi; ++i)
        {
            const int64_t slot = static_cast<int64_t>(i) + b;
            const float   w = __builtin_amdgcn_exp2f(a.ws_ml[(slot * a.num_heads + h) * 2] - M);
            lsum += a.ws_ml[(slot * a.num_heads + h) * 2 + 1] * w;
            o += a.ws_acc[(slot * a.num_heads + h) * D + d] * w;
        }
    }
    store_act1(a.out, QT, oi, lsum > 0.0f ? o / lsum : 0.0f);
}

namespace
{

template <int CT, int QT, int D>
hipError_t launch_m3(const DecodeArgs& a0, hipStream_t stream)
{
    DecodeArgs a = a0;
    const int  nw = a.num_kv_heads < 4 ? a.num_kv_heads : 4;
    const int  gy = (a.num_kv_heads + nw - 1) / nw;
    const auto kern = paged_decode_mfma<CT, QT, D>;
    const int  items = decode_mfma_items(reinterpret_cast<const void*>(kern), 64 * nw, gy);
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(items), static_cast<unsigned>(gy)), dim3(64 * nw), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    constexpr int HPW = 256 / D;
    hipLaunchKernelGGL((paged_decode_mfma_merge<QT, D>),
                       dim3(static_cast<unsigned>(a.batch), static_cast<unsigned>((a.num_heads + HPW - 1) / HPW)),
                       dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <int CT, int QT>
hipError_t launch_m2(const DecodeArgs& a, hipStream_t stream)
{
    switch (a.head_dim)
    {
        case 64:
            return launch_m3<CT, QT, 64>(a, stream);
        case 128:
            return launch_m3<CT, QT, 128>(a, stream);
        default:
            return launch_m3<CT, QT, 256>(a, stream);
    }
}

template <int CT>
hipError_t launch_m1(const DecodeArgs& a, hipStream_t stream)
{
    switch (a.qo_dtype)
    {
        case F32:
            return launch_m2<CT, F32>(a, stream);
        case F16:
            return launch_m2<CT, F16>(a, stream);
        default:
            return launch_m2<CT, BF16>(a, stream);
    }
}

}  // namespace

hipError_t launch_decode_mfma(const DecodeArgs& a, hipStream_t stream)
{
    switch (a.cache_dtype)
    {
        case BF16:
            return launch_m1<BF16>(a, stream);
        case F16:
            return launch_m1<F16>(a, stream);
        case I8:
            return launch_m1<I8>(a, stream);
        default:
            return launch_m1<FP8>(a, stream);
    }
}

}  // namespace ffkv
