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
//     layout (k = token = 4g + i), V^T comes from an LDS copy of the page's V rows whose 16-byte chunks are
//     XOR-swizzled per token, so both the 16-byte row writes and the transposing column reads are free of bank
//     conflicts while every row stays 16-byte aligned.
//     P is split into hi + lo parts of the MFMA input type, so the products carry ~16 significant bits.
//   * quantized caches: int8 and fp8 e4m3 codes convert exactly to f16 for the MFMA; int8 per-token K scales
//     multiply the scores and V scales multiply P, fp8 per-head scales fold into the score scale and the output.
//   * work split: the pages of all rows form one sequence; work item i of W takes pages
//     [i*P/W, (i+1)*P/W), so every wave gets the same number of pages whatever the row lengths (no tail of
//     long rows).  A row covered by one item writes its output directly; otherwise each piece writes an
//     unnormalised partial (m, l, acc) to slot item + row and paged_decode_mfma_merge combines them.
#include "ffkv_device.h"
#include "ffkv_internal.h"

#ifndef FFKV_MFMA_MAX_WAVES
#define FFKV_MFMA_MAX_WAVES 4  // waves (= KV heads) per workgroup
#endif

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
    // v_cvt_pk_bf16_f32: round to nearest even (the operands here are finite)
    static __device__ __forceinline__ uint32_t bits(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }
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

using h2 = _Float16 __attribute__((ext_vector_type(2)));

// 4 int8 codes -> 4 f16 values (two packed words), exact: the biased byte u = code + 128 is placed under the f16
// exponent of 1024 (0x64uu = 1024 + u) and 1152 is subtracted with one packed f16 add per pair.
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi)
{
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [u0, 0x64, u1, 0x64]
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [u2, 0x64, u3, 0x64]
    const h2       bias = h2{static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) + bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, b) + bias);
}

// 4 OCP e4m3 codes -> 4 f16 values, exact: the code's magnitude bits shifted into the f16 exponent/mantissa
// fields give 2^-8 times the value (normal and subnormal alike), fixed by one packed multiply by 256; the
// NaN codes (S.1111.111) become f16 NaN.
__device__ __forceinline__ void fp8x4_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi)
{
    const uint32_t x0 = __builtin_amdgcn_perm(0u, w, 0x010c000cu);  // [0, b0, 0, b1]
    const uint32_t x1 = __builtin_amdgcn_perm(0u, w, 0x030c020cu);  // [0, b2, 0, b3]
    const uint32_t f0 = (x0 & 0x80008000u) | ((x0 >> 1) & 0x3f803f80u);
    const uint32_t f1 = (x1 & 0x80008000u) | ((x1 >> 1) & 0x3f803f80u);
    const h2       k256 = h2{static_cast<_Float16>(256.0f), static_cast<_Float16>(256.0f)};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, f0) * k256);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, f1) * k256);
    // a byte whose low 7 bits are all ones is NaN; (b & 0x7f) + 1 carries into bit 7 only for those
    const uint32_t nan = ((w & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;
    if (__builtin_expect(nan != 0u, 0))
    {
        const uint32_t n0 = __builtin_amdgcn_perm(0u, nan, 0x010c000cu);  // NaN flags at bit 15 of each half
        const uint32_t n1 = __builtin_amdgcn_perm(0u, nan, 0x030c020cu);
        lo = (lo & ~(((n0 >> 15) & 0x00010001u) * 0x7fffu)) | (((n0 >> 15) & 0x00010001u) * 0x7e00u);
        hi = (hi & ~(((n1 >> 15) & 0x00010001u) * 0x7fffu)) | (((n1 >> 15) & 0x00010001u) * 0x7e00u);
    }
}

// 8 cache codes (one k-step of one lane) as 4 packed 16-bit MFMA words.  Quantized codes convert exactly.
template <int CT>
__device__ __forceinline__ u32x4 codes_to_m(uint32_t lo, uint32_t hi)
{
    uint32_t r0, r1, r2, r3;
    if constexpr (CT == I8)
    {
        i8x4_to_f16(lo, r0, r1);
        i8x4_to_f16(hi, r2, r3);
    }
    else
    {
        fp8x4_to_f16(lo, r0, r1);
        fp8x4_to_f16(hi, r2, r3);
    }
    return u32x4{r0, r1, r2, r3};
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
        for (int k = 0; k < 4; ++k)
            h[k] = QT == BF16 ? __builtin_bit_cast(uint16_t, static_cast<__bf16>(v[k]))
                              : __builtin_bit_cast(uint16_t, static_cast<_Float16>(v[k]));
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

// Registers of one loaded page, as loaded: NW 16-byte words of K and of V per lane (one k-step each for 16-bit
// caches, two for 8-bit codes, which convert when the page is staged so the loads stay in flight until then).
template <int NW>
struct PageRegs
{
    u32x4 k[NW];
    u32x4 v[NW];
    int   phys;
    bool  ok;
};

// Position (16-bit elements) of V[t][d] in a wave's LDS tile of 16 rows x D.  The 16-byte chunk d/8 of row t
// is stored at chunk (d/8) ^ sw(t) with sw(t) = (t % 8) ^ 2 * (t / 8).  Both access patterns then hit distinct
// bank groups: a 16-byte write by 8 consecutive lanes (8 tokens, same chunk) spreads over 8 chunk slots mod 8,
// and a PV operand read (tokens 4g + i for g = 0..3, chunks 2n and 2n + 1) touches 8 distinct slots mod 8.
template <int D>
__device__ __forceinline__ int lds_pos(int t, int d)
{
    const int sw = (t & 7) ^ ((t >> 3) << 1);
    return t * D + ((((d >> 3) ^ sw)) << 3) + (d & 7);
}

__device__ __forceinline__ int wave_sum(int x)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

// A value equal in all lanes, moved to a scalar register.
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

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

// Waves per SIMD the register budget is sized for, with one page's K/V in flight beside the page being finished:
// 3 (168 registers) at D = 128, 4 (128) at D = 64, 2 at D = 256.
template <int CT, int QT, int D>
constexpr int kMfmaWaves = D == 256 ? 2 : (D == 128 ? 3 : 4);

// Work item i (blockIdx.x) of W (gridDim.x); KV heads blockIdx.y*NW .. +NW, one per wave.
template <int CT, int QT, int D>
__global__ __launch_bounds__(64 * FFKV_MFMA_MAX_WAVES) __attribute__((amdgpu_waves_per_eu(kMfmaWaves<CT, QT, D>, 8)))
void paged_decode_mfma(DecodeArgs a)
{
    constexpr bool BF = kBF<CT>;
    using M = MType<BF>;
    using X8 = typename M::x8;
    constexpr int  KSTEPS = D / 32;
    constexpr int  NT = D / 16;  // output tiles of 16 dims
    constexpr bool NEED_LO = !((QT == BF16 && BF) || (QT == F16 && !BF));

    __shared__ uint16_t s_v[FFKV_MFMA_MAX_WAVES][kBlockSize * D];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c = lane & 15;  // MFMA column / row-in-tile index
    const int g = lane >> 4;  // lane group
    const int B = a.batch;
    const bool first_wg = blockIdx.x == 0 && blockIdx.y == 0 && wave == 0;

    // ---- total pages P, each wave on its own (64 rows per pass, no barriers) -----------------------------
    // Rows without any token get a zero output and "no pieces" meta here; nothing else touches them.
    // Page counts fit in 32 bits: the host bounds batch * pages per row.
    int P = 0;
    for (int r0 = 0; r0 < B; r0 += 64)
    {
        const int r = r0 + lane;
        const int n = r < B ? row_pages(a, r) : 0;
        P += uniform(wave_sum(n));
        if (first_wg && r < B && n == 0)
        {
            for (int e = 0; e < a.num_heads * D; e += 4)
                store_out4<QT>(a.out, static_cast<size_t>(r) * a.num_heads * D + e, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
            a.ws_meta[2 * r] = -1;
            a.ws_meta[2 * r + 1] = -1;
        }
    }
    const int W = min(static_cast<int>(gridDim.x), P);
    const int item = blockIdx.x;
    if (item >= W) return;
    const int start = static_cast<int>(static_cast<int64_t>(item) * P / W);
    const int end = static_cast<int>(static_cast<int64_t>(item + 1) * P / W);

    // ---- row holding page `start`: second pass with an inclusive wave scan ------------------------------
    int b0 = 0;
    int pb0 = 0;
    for (int r0 = 0; r0 < B; r0 += 64)
    {
        const int r = r0 + lane;
        const int n = r < B ? row_pages(a, r) : 0;
        int       incl = n;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1)
        {
            const int o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        const uint64_t hit = __ballot(pb0 + incl - n <= start && start < pb0 + incl);
        if (hit != 0)
        {
            const int l = __ffsll(static_cast<long long>(hit)) - 1;
            b0 = r0 + l;
            pb0 += uniform(__shfl(incl - n, l, 64));
            break;
        }
        pb0 += uniform(__shfl(incl, 63, 64));
    }

    const int kvh = blockIdx.y * (static_cast<int>(blockDim.x) >> 6) + wave;
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

    // ---- per-row state ------------------------------------------------------------------------------------
    struct Row
    {
        int            b;
        int            pb;  // global index of the row's first page
        int            nb;  // pages in the row
        int            Lp;  // attended tokens
        const int32_t* table;
    };
    auto make_row = [&](int b, int pb)
    {
        return Row{b, pb, row_pages(a, b), row_tokens(a, b), a.block_table + static_cast<int64_t>(b) * a.max_blocks};
    };
    auto next_row = [&](const Row& r)
    {
        const int pb = r.pb + r.nb;
        int       b = r.b + 1;
        while (row_pages(a, b) == 0) ++b;
        return make_row(b, pb);
    };

    X8   qhi[KSTEPS], qlo[KSTEPS];
    auto load_q = [&](int b)  // Q of row b's group as MFMA B operands (column c = head, zero beyond the group)
    {
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
            if constexpr (!NEED_LO)
            {
                // q is stored in the MFMA input type: its 16 bytes are the operand
                u32x4 w = u32x4{0u, 0u, 0u, 0u};
                if (c < G)
                    w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.q) +
                                                        (static_cast<size_t>(b) * a.num_heads + kvh * G + c) * D +
                                                        dim_of<CT>(j, g));
                qhi[j] = __builtin_bit_cast(X8, w);
                qlo[j] = qhi[j];
            }
            else
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
                    lo[e] = M::bits(x[e] - M::value(hi[e]));
                }
                qhi[j] = __builtin_bit_cast(X8, u32x4{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16),
                                                      hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16)});
                qlo[j] = __builtin_bit_cast(X8, u32x4{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16),
                                                      lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16)});
            }
        }
    };

    float m_run = kNegInf;  // running max of head c (log2 domain), equal in the four lane groups
    float l_run = 0.0f;     // this lane's share of the denominator (tokens 4g..4g+3 of each page)
    f32x4 acc[NT];

    // Issue the K and V loads of physical page `phys` (token c of the page, lane group g's dims) into registers.
    constexpr int NW = kElemBytes<CT> == 2 ? KSTEPS : KSTEPS / 2;
    auto          load_page = [&](int phys, PageRegs<NW>& r)
    {
        r.phys = phys;
        r.ok = phys >= 0 && phys < a.num_blocks;  // uniform: a masked page is skipped
        if (!r.ok) return;
        const size_t row_c = (static_cast<size_t>(phys) * kBlockSize + c) * a.num_kv_heads + kvh;
        if constexpr (kElemBytes<CT> == 2)
        {
            const char* kp = static_cast<const char*>(a.k_cache) + row_c * D * 2;
            const char* vp = static_cast<const char*>(a.v_cache) + row_c * D * 2;
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j)
            {
                r.k[j] = *reinterpret_cast<const u32x4*>(kp + dim_of<CT>(j, g) * 2);
                r.v[j] = *reinterpret_cast<const u32x4*>(vp + dim_of<CT>(j, g) * 2);
            }
        }
        else
        {
            const char* kp = static_cast<const char*>(a.k_cache) + row_c * D;
            const char* vp = static_cast<const char*>(a.v_cache) + row_c * D;
#pragma unroll
            for (int j = 0; j < KSTEPS; j += 2)
            {
                r.k[j / 2] = *reinterpret_cast<const u32x4*>(kp + dim_of<CT>(j, g));
                r.v[j / 2] = *reinterpret_cast<const u32x4*>(vp + dim_of<CT>(j, g));
            }
        }
    };

    // Stage a loaded page: V rows into the wave's LDS tile, scores S^T = K Q^T into s.  Consumes r.k and r.v,
    // so the next page can be loaded into r right after.
    // K or V words of k-step j in the MFMA input type.
    auto mword = [&](const u32x4* w, int j) -> u32x4
    {
        if constexpr (kElemBytes<CT> == 2)
            return w[j];
        else
            return (j & 1) ? codes_to_m<CT>(w[j / 2][2], w[j / 2][3]) : codes_to_m<CT>(w[j / 2][0], w[j / 2][1]);
    };
    auto stage_page = [&](int n_tok, const PageRegs<NW>& r, f32x4& s)
    {
        const bool tok_ok = c < n_tok;  // V[t = c], zero for slots past the row's last token
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
            const u32x4 w = tok_ok ? mword(r.v, j) : u32x4{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4*>(sv + lds_pos<D>(c, dim_of<CT>(j, g))) = w;
        }
        s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};  // lane (c, g) gets tokens 4g + i of head c
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
            const X8 kj = __builtin_bit_cast(X8, mword(r.k, j));
            s = M::mma32(kj, qhi[j], s);
            if constexpr (NEED_LO) s = M::mma32(kj, qlo[j], s);
        }
    };

    // Online softmax of a staged page's scores and PV from its LDS tile.
    auto finish_page = [&](int n_tok, int phys, f32x4 s)
    {
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
        const typename M::x4 phi =
            __builtin_bit_cast(typename M::x4, u32x2{ph[0] | (ph[1] << 16), ph[2] | (ph[3] << 16)});
        const typename M::x4 plo =
            __builtin_bit_cast(typename M::x4, u32x2{pl[0] | (pl[1] << 16), pl[2] | (pl[3] << 16)});

        // LDS writes of this wave are complete before its reads below (in-order LDS queue of one wave);
        // the fence keeps the compiler from moving the reads above the writes.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // O^T[d, h] += V^T[d, t] P^T[t, h] over the 16 dims of each tile
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
    };

    // Write the segment [seg_start, seg_end) of row `row`: the output if it is the whole row, else a partial.
    auto finish_segment = [&](const Row& row, int seg_start, int seg_end)
    {
        const float l_tot = xor_sum(l_run);
        const int   h = kvh * G + c;
        if (seg_start == row.pb && seg_end == row.pb + row.nb)
        {
            if (c < G)
            {
                const float inv = l_tot > 0.0f ? v_head_scale / l_tot : 0.0f;
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    store_out4<QT>(a.out, (static_cast<size_t>(row.b) * a.num_heads + h) * D + 16 * n + 4 * g,
                                   acc[n] * inv);
            }
        }
        else if (c < G)
        {
            const int64_t slot = static_cast<int64_t>(item) + row.b;
            float*        dst = a.ws_acc + (slot * a.num_heads + h) * D;
#pragma unroll
            for (int n = 0; n < NT; ++n)
                *reinterpret_cast<f32x4*>(dst + 16 * n + 4 * g) = acc[n] * v_head_scale;
            if (g == 0)
            {
                a.ws_ml[(slot * a.num_heads + h) * 2] = m_run;
                a.ws_ml[(slot * a.num_heads + h) * 2 + 1] = l_tot;
            }
        }
        // the item holding a row's first page records which items cover the row
        if (seg_start == row.pb && blockIdx.y == 0 && wave == 0 && lane == 0)
        {
            const int64_t last = row.pb + row.nb - 1;
            const int64_t i_hi = ((last + 1) * W + P - 1) / P - 1;  // largest i with i*P/W <= last
            a.ws_meta[2 * row.b] = item;
            a.ws_meta[2 * row.b + 1] = static_cast<int32_t>(i_hi);
        }
    };

    // ---- one flat pass over the item's pages ------------------------------------------------------------
    // The loads of page p + 1 are issued as soon as page p's registers are consumed and stay in flight during
    // page p's softmax and PV - across row boundaries too: the next row, its first block-table entry and its Q
    // are fetched ahead, so a row change costs no extra memory round trip.
    Row     cur = make_row(b0, pb0);
    Row     nxt = cur;
    int     nxt_phys0 = -1;
    int     seg_start = start;
    auto    begin_segment = [&]()
    {
        m_run = kNegInf;
        l_run = 0.0f;
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (cur.pb + cur.nb < end)
        {
            nxt = next_row(cur);
            nxt_phys0 = nxt.table[0];
        }
    };
    load_q(cur.b);
    begin_segment();
    PageRegs<NW> r;
    load_page(cur.table[start - cur.pb], r);
    for (int p = start; p < end; ++p)
    {
        const int  pg = static_cast<int>(p - cur.pb);
        const int  n_tok = min(kBlockSize, cur.Lp - pg * kBlockSize);
        const bool ok = r.ok;
        const int  phys = r.phys;
        const bool row_ends = p + 1 == cur.pb + cur.nb;
        f32x4      s;
        if (ok) stage_page(n_tok, r, s);
        if (p + 1 < end)
        {
            load_page(row_ends ? nxt_phys0 : cur.table[pg + 1], r);
            if (row_ends) load_q(nxt.b);  // the scores of page p have consumed Q
        }
        if (ok) finish_page(n_tok, phys, s);
        if (row_ends || p + 1 == end)
        {
            finish_segment(cur, seg_start, p + 1);
            if (p + 1 < end)
            {
                cur = nxt;
                seg_start = p + 1;
                begin_segment();
            }
        }
    }
}

// Combine the partials of rows split over several work items.
// One workgroup of four waves per (row, head): wave w folds segments i_lo + w, i_lo + w + 4, ... into an online
// (max, denominator, output) state (lane = D/64 dims), then the four states are combined through LDS.
template <int QT, int D>
__global__ __launch_bounds__(256) void paged_decode_mfma_merge(DecodeArgs a)
{
    constexpr int PER = D / 64;  // dims per lane
    const int     b = blockIdx.x;
    const int     h = blockIdx.y;
    const int     lane = threadIdx.x & 63;
    const int     wave = threadIdx.x >> 6;
    const size_t  ob = (static_cast<size_t>(b) * a.num_heads + h) * D;
    __shared__ float s_m[4], s_l[4];
    __shared__ float s_o[4][D];

    const int i_lo = a.ws_meta[2 * b];
    const int i_hi = a.ws_meta[2 * b + 1];
    if (i_lo == i_hi) return;  // one piece (written by the decode kernel) or no token (i_lo = i_hi = -1)

    float m = kNegInf, l = 0.0f, o[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) o[k] = 0.0f;
    for (int i = i_lo + wave; i <= i_hi; i += 4)
    {
        const int64_t slot = static_cast<int64_t>(i) + b;
        const float   ms = a.ws_ml[(slot * a.num_heads + h) * 2];
        const float   ls = a.ws_ml[(slot * a.num_heads + h) * 2 + 1];
        const float*  src = a.ws_acc + (slot * a.num_heads + h) * D + lane * PER;
        float         x[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) x[k] = src[k];
        if (ms == kNegInf) continue;  // segment without a valid page
        const float mn = fmaxf(m, ms);
        const float wa = __builtin_amdgcn_exp2f(m - mn);
        const float wb = __builtin_amdgcn_exp2f(ms - mn);
        l = l * wa + ls * wb;
#pragma unroll
        for (int k = 0; k < PER; ++k) o[k] = o[k] * wa + x[k] * wb;
        m = mn;
    }
    if (lane == 0)
    {
        s_m[wave] = m;
        s_l[wave] = l;
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) s_o[wave][lane * PER + k] = o[k];
    __syncthreads();
    if (threadIdx.x < D)
    {
        const int d = threadIdx.x;
        float     M = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
        float     L = 0.0f, O = 0.0f;
        if (M != kNegInf)
        {
#pragma unroll
            for (int w = 0; w < 4; ++w)
            {
                const float wt = __builtin_amdgcn_exp2f(s_m[w] - M);
                L += s_l[w] * wt;
                O += s_o[w][d] * wt;
            }
        }
        store_act1(a.out, QT, ob + d, L > 0.0f ? O / L : 0.0f);
    }
}

namespace
{

template <int CT, int QT, int D>
hipError_t launch_m3(const DecodeArgs& a0, hipStream_t stream)
{
    DecodeArgs a = a0;
    const int  nw = a.num_kv_heads < FFKV_MFMA_MAX_WAVES ? a.num_kv_heads : FFKV_MFMA_MAX_WAVES;
    const int  gy = (a.num_kv_heads + nw - 1) / nw;
    const auto kern = paged_decode_mfma<CT, QT, D>;
    const int  items = decode_mfma_items(reinterpret_cast<const void*>(kern), 64 * nw, gy);
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(items), static_cast<unsigned>(gy)), dim3(64 * nw), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((paged_decode_mfma_merge<QT, D>),
                       dim3(static_cast<unsigned>(a.batch), static_cast<unsigned>(a.num_heads)), dim3(256), 0, stream, a);
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
