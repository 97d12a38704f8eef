// paged_decode_mfma.hip - PagedAttention decode on the gfx950 matrix cores, split evenly over pages.
//
// Reference semantics: paged_attention_kernel (src/kernels/attention.cu:291-447): out[b, h] = softmax over the
// context_lens[b] + 1 cached tokens of scale * q[b, h] . k_j, applied to v_j, with kv_head = h / (Hq / Hkv).
//
// Design (one wave = one KV head of one page range, or one block of 16 of its query heads when the GQA group is
// larger; a page = 16 tokens = one MFMA tile):
//   * QK^T on MFMA: S^T[t, h] = K[t, :] . Q[h, :] with v_mfma_f32_16x16x32_{bf16,f16}; the 16 tokens of a page
//     are the rows, (up to) 16 query heads of the GQA group the columns.  Groups over 16 heads take one wave per
//     block of 16; the blocks of a KV head sit in the same workgroup, so their reads of a page meet in L2.  K is fed straight from its page:
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
//     bf16 P is split into hi + lo parts, so the products carry ~16 significant bits; f16 P (f16 caches, and the
//     f16 PV products of 8-bit caches) is one product of 11 bits.
//   * quantized caches: int8 and fp8 e4m3 codes convert exactly to the MFMA input type when a page is staged
//     (fp8 with the gfx950 conversion instructions, int8 with byte permutes and packed f16 ops); int8 per-token
//     K scales multiply the scores and V scales multiply P, fp8 per-head scales fold into the score scale and
//     the output.
//   * work split: the pages of all rows form one sequence; work item i of W takes pages
//     [i*P/W, (i+1)*P/W), so every wave gets the same number of pages whatever the row lengths (no tail of
//     long rows).  A row covered by one item writes its output directly; otherwise each piece writes an
//     unnormalised partial (m, l, acc) to slot item + row and paged_decode_mfma_merge combines them.
//   * streaming: a load cursor runs DEPTH pages ahead of the page being finished, across row boundaries.  Rows
//     are found with ballots over windows of 64 rows held one per lane (one vector load of context_lens per
//     window), block-table entries come 64 per vector load, and the next row's Q is loaded as soon as the last
//     page of a row has been scored, so a wave never waits on a dependent scalar load between pages.
#include "mfma_common.h"

#ifndef FFKV_MERGE_ROWS_MIN_BATCH
#define FFKV_MERGE_ROWS_MIN_BATCH 16  // batches above this merge with paged_decode_mfma_merge_rows
#endif

#ifndef FFKV_MFMA_MAX_WAVES
#define FFKV_MFMA_MAX_WAVES 4  // waves (KV heads, or blocks of 16 query heads of one) per workgroup
#endif
#ifndef FFKV_MFMA_MAX_WAVES_WIDE
#define FFKV_MFMA_MAX_WAVES_WIDE 8  // the same for 16-bit caches at head_dim 96 and fp8 caches at 128
#endif

namespace ffkv
{

namespace
{

// One page in flight: NW 16-byte words of K per lane as loaded (one k-step each for 16-bit caches, two for 8-bit
// codes, which convert when the page is staged so the loads stay in flight until then), the K words of a last
// 16-dim k-step (head_dim 80, 112), NWV 16-byte words of V, the physical block, and the row the page belongs to.
template <int NW, int NWV>
struct PageRegs
{
    u32x4 k[NW > 0 ? NW : 1];
    u32x2 kt;  // last 16-dim k-step: 4 values (8 bytes) of 16-bit K, or 4 codes (first word)
    u32x4 v[NWV];
    int   phys;
    bool  ok;
    int   b;   // row
    int   pb;  // global index of the row's first page
    int   nb;  // pages of the row
    int   lp;  // attended tokens of the row
    int   ns;  // fused append: slot of the row's new token in this page, else -1
    float ks;  // int8 caches: K and V scale of token c (lane c of each lane group)
    float vs;
};

}  // namespace

#ifndef FFKV_MFMA_DEPTH16
#define FFKV_MFMA_DEPTH16 2  // pages in flight per wave: 16-bit caches
#endif
#ifndef FFKV_DECODE_V16
#define FFKV_DECODE_V16 1  // 8-bit caches: PV products in f16 (P in one product)
#endif

#ifndef FFKV_MFMA_DEPTH_FP8
#define FFKV_MFMA_DEPTH_FP8 2  // fp8 caches
#endif
#ifndef FFKV_MFMA_DEPTH_I8
#define FFKV_MFMA_DEPTH_I8 1  // int8 caches
#endif
#ifndef FFKV_MFMA_WAVES128_16
#define FFKV_MFMA_WAVES128_16 (FFKV_MFMA_DEPTH16 > 1 ? 2 : 3)
#endif
#ifndef FFKV_MFMA_WAVES128_FP8
#define FFKV_MFMA_WAVES128_FP8 (FFKV_MFMA_DEPTH_FP8 > 1 ? 2 : 3)
#endif
#ifndef FFKV_MFMA_WAVES128_I8
#define FFKV_MFMA_WAVES128_I8 3
#endif

#ifndef FFKV_MFMA_DEPTH256
#define FFKV_MFMA_DEPTH256 1  // head_dim 256: a page in flight is 64 registers (16-bit), two would spill
#endif

// Pages whose K/V loads are in flight while a wave finishes the page before them.
template <int CT, int D>
constexpr int kMfmaDepth =
    D == 256 ? FFKV_MFMA_DEPTH256
             : (kElemBytes<CT> == 2 ? FFKV_MFMA_DEPTH16 : (CT == FP8 ? FFKV_MFMA_DEPTH_FP8 : FFKV_MFMA_DEPTH_I8));

#ifndef FFKV_MFMA_WAVES80
#define FFKV_MFMA_WAVES80 2  // head_dim 80 with q in the cache's type (three waves' 168 registers spill)
#endif

// Waves per SIMD the register budget is sized for (168 registers at 3, 128 at 4, 256 at 2).
template <int CT, int QT, int D>
constexpr int kMfmaWaves =
    D == 256 || D == 112 ? 2
    : D == 96 ? (QT == CT ? 3 : 2)  // a q of another type needs its lo part: three waves' registers would spill
    : D == 80 ? (QT == CT ? FFKV_MFMA_WAVES80 : 2)
             : (D == 128 ? (kElemBytes<CT> == 2 ? FFKV_MFMA_WAVES128_16
                                                : (CT == FP8 ? FFKV_MFMA_WAVES128_FP8 : FFKV_MFMA_WAVES128_I8))
                         : (kMfmaDepth<CT, D> > 1 ? 3 : 4));


// Page loads.  V is staged through LDS, so its loads can take any lane layout: each load instruction reads 64
// consecutive 16-byte chunks of the wave's slice of the page (whole 128-byte lines of 4 token rows at head_dim
// 128), non-temporal.  K feeds the matrix products straight from its registers, so its lanes keep the operand
// layout (64 bytes of each of 16 token rows per instruction).  A read-only stream measured 6.3 TB/s with plain
// loads in either layout and 7.0-7.2 TB/s once the whole-line half of the traffic is non-temporal: pages are read
// once per call, and plain loads also allocate them in the caches on the way.
#ifndef FFKV_DECODE_NT_V
#define FFKV_DECODE_NT_V 1
#endif
#ifndef FFKV_DECODE_TIMELINE
#define FFKV_DECODE_TIMELINE 0  // 1: each wave of the split-K kernel records its start and end (timeline builds)
#endif
#ifndef FFKV_DECODE_NT_K
#define FFKV_DECODE_NT_K 0  // K (the operand-layout half) non-temporal too
#endif

template <bool NT>
__device__ __forceinline__ u32x4 load16(const char* p)
{
    if constexpr (NT)
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    else
        return *reinterpret_cast<const u32x4*>(p);
}

// Position of element (token t, dim d) of a wave's V tile: 16-byte chunks XOR-swizzled by row so that the four
// rows of one transposed read (two chunks each) sit on distinct banks.
// Bit 0 of the chunk index is also flipped for the chunks written by lanes 4..7 of each group of 8 (flip below):
// a scattered 16-byte LDS write is served 8 lanes at a time over 128 bytes, and an 8-bit page's lane writes the
// 8 values of its first half to chunk 2ch and those of its second half to 2ch + 1 (16 codes, dims 16 ch ..
// 16 ch + 15), so without the flip the 8 lanes of a group would fill chunks of one parity only, two lanes per
// bank group.  A flip only swaps the two chunks of a 16-dim pair, which a transposed read takes together.
template <int D>
__device__ __forceinline__ int vt_pos(int t, int d)
{
    // 16 codes per chunk of an 8-bit page: lane group bit of the code chunk (row t, 16-dim pair d / 16)
    const int flip = ((t * (D / 16) + (d >> 4)) >> 2) & 1;
    // head_dim 96 (12 chunks a row, whose 192-byte stride already spreads a read's four rows over the banks): the
    // swizzle stays within aligned groups of four chunks, so it never leaves the row; head_dim 80 and 112 (160- and
    // 224-byte rows) put the 8 rows of two transposed reads on distinct banks unswizzled
    const int sw = D == 80 || D == 112 ? 0 : (D == 64 ? 2 * ((t >> 1) & 3) : (D == 96 ? 2 * ((t >> 2) & 1) : 2 * (t & 7)));
    return t * D + (((d >> 3) ^ sw ^ flip) << 3) + (d & 7);
}

// Waves per workgroup (the KV heads, or blocks of 16 query heads, that read the same pages together).  With 8
// (all 8 KV heads of a Qwen-shaped page) the whole page is fetched by one workgroup at once: C2-shaped decode at
// head_dim 96 98.6 -> 88.8 us, fp8 C5 395 -> 390 us; bf16 at 128 unchanged, int8 slower (417 -> 439 us).
template <int CT, int D>
constexpr int kMfmaMaxWaves =
    ((D == 80 || D == 96 || D == 112) && kElemBytes<CT> == 2) || (CT == FP8 && D == 128) ? FFKV_MFMA_MAX_WAVES_WIDE
                                                                                          : FFKV_MFMA_MAX_WAVES;

// One workgroup of a decode launch: work item `item` of `n_items`, KV heads y*nw .. +nw (one per wave; nw waves
// in the workgroup).  s_v: the workgroup's V tiles in LDS, [nw][16 * D] 16-bit elements.  PW: the page split may
// weigh the first pfx_items items less (the fused shared-prefix launch); the plain decode's split otherwise.
template <int CT, int QT, int D, bool PW = false>
__device__ __forceinline__ void decode_wg(const DecodeArgs& a, int item_, int y_, int n_items_, int nw_, uint16_t* s_v)
{
    // (the plain decode reads its indices where it uses them: held in registers from the start, they cost the
    // kernel scalar registers it spills)
    auto item_of = [&]() { return PW ? item_ : static_cast<int>(blockIdx.x); };
    auto y_of = [&]() { return PW ? y_ : static_cast<int>(blockIdx.y); };
    // Score products in M (BF: bf16, else f16); PV products in MV.  8-bit codes are exact in both types, so their
    // PV products take f16, where P fits one product (11 bits) instead of a bf16 hi + lo pair; bf16 caches keep
    // bf16 P as hi + lo.  (int8 scores stay f16 with q split in two: bf16 scores, q whole, measured 20 % slower
    // on C5 from the extra conversion registers.)
    constexpr bool BF = kBF<CT, QT>;
    constexpr bool VBF = CT == BF16 || (kElemBytes<CT> == 1 && BF && !FFKV_DECODE_V16);
    using M = MType<BF>;
    using MV = MType<VBF>;
    using X8 = typename M::x8;
    using X4 = typename M::x4;
    constexpr int  KSTEPS = D / 32;            // k-steps of 32 dims (16x16x32 products)
    constexpr bool KT = D % 32 == 16;          // and a last one of 16 dims (16x16x16): head_dim 80, 112
    constexpr int  DT = 32 * KSTEPS;           // its first dim
    constexpr int  NT = D / 16;  // output tiles of 16 dims
    constexpr bool NEED_LO = !((QT == BF16 && BF) || (QT == F16 && !BF));
    constexpr bool P_LO = VBF;  // bf16 P: hi + lo parts
    constexpr int  DEPTH = kMfmaDepth<CT, D>;
    constexpr int  NW = kElemBytes<CT> == 2 ? KSTEPS : (KSTEPS + 1) / 2;
    constexpr int  VCPR = D * kElemBytes<CT> / 16;  // 16-byte chunks of a token's V row
    constexpr int  NWV = (kBlockSize * VCPR + 63) / 64;  // V load instructions per page
    // First dim of k-step j's 8 values in lane group g.  8-bit codes pair k-steps in one 16-byte read; an odd last
    // k-step (head_dim 96) reads its 8 codes alone, at dims 32j + 8g.
    auto dimof = [](int j, int g)
    {
        if constexpr (kElemBytes<CT> == 1 && KSTEPS % 2 == 1)
            if (j == KSTEPS - 1) return 32 * j + 8 * g;
        return dim_of<CT>(j, g);
    };

    const int  lane = threadIdx.x & 63;
    const int  wave = threadIdx.x >> 6;
    const int  c = lane & 15;  // MFMA column / row-in-tile index
    const int  g = lane >> 4;  // lane group
    const int  B = a.batch;
    const bool first_wg = item_of() == 0 && y_of() == 0 && wave == 0;

    // ---- rows in windows of 64, one row per lane --------------------------------------------------------------
    // A window holds rows w0 .. w0 + 63: lane l has row w0 + l's attended tokens, pages and first page (relative to
    // the window's first page `base`); `total` is the window's page count.  Rows are located with ballots over a
    // window instead of memory reads; a new window costs one vector load of context_lens.
    struct Win
    {
        int w0, base, total;
        int toks, n, excl;  // per lane
        int whole;          // per lane: the row's new token (position context_lens) is attended (not truncated)
    };
    auto load_win = [&](int w0, int base)
    {
        const int r = w0 + lane;
        int       t = 0;
        int       whole = 0;
        if (r < B)
        {
            int64_t L = static_cast<int64_t>(a.context_lens[r]) + 1;  // +1: the token appended this step (:320)
            whole = L <= a.cap_tokens;
            if (L > a.cap_tokens) L = a.cap_tokens;
            t = L < 0 ? 0 : static_cast<int>(L);
        }
        // shared-prefix mode: the row's first skip_blocks pages are attended elsewhere
        int n = (t + kBlockSize - 1) / kBlockSize - a.skip_blocks;
        n = n < 0 ? 0 : n;
        t = t - a.skip_blocks * kBlockSize;
        t = t < 0 ? 0 : t;
        int incl = n;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1)
        {
            const int o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        return Win{w0, base, uniform(__shfl(incl, 63, 64)), t, n, incl - n, whole};
    };

    // ---- total pages P (every wave on its own, no barriers) -------------------------------------------------
    // Rows without any token get a zero output and "no pieces" meta here; nothing else touches them.
    const Win win0 = load_win(0, 0);
    int       P = 0;
    for (Win w = win0;;)
    {
        if (first_wg && w.w0 + lane < B && w.n == 0)
        {
            const int r = w.w0 + lane;
            if (a.pfx_chunks == 0)  // shared-prefix mode: the merge writes every row
                for (int e = 0; e < a.num_heads * D; e += 4)
                    store_out4<QT>(a.out, static_cast<size_t>(r) * a.num_heads * D + e,
                                   f32x4{0.0f, 0.0f, 0.0f, 0.0f});
            a.ws_meta[2 * r] = -1;
            a.ws_meta[2 * r + 1] = -1;
        }
        if constexpr (kElemBytes<CT> == 2)
        {
            // Fused append, rows cut short by max_context_len: their new token is not attended, so no page
            // holding it is staged; the first wave copies it to its slot here, as ffkv_append would.
            uint64_t cut = first_wg && a.k_new != nullptr ? __ballot(w.w0 + lane < B && !w.whole) : 0;
            while (cut != 0)
            {
                const int r = w.w0 + __ffsll(static_cast<long long>(cut)) - 1;
                cut &= cut - 1;
                const int64_t pos = a.context_lens[r];
                if (pos < 0 || (pos >> 4) >= a.max_blocks) continue;
                const int phys = a.block_table[static_cast<int64_t>(r) * a.max_blocks + (pos >> 4)];
                if (phys < 0 || phys >= a.num_blocks) continue;
                const size_t dst = (static_cast<size_t>(phys) * kBlockSize + (pos & 15)) * a.num_kv_heads * D;
                const size_t src = static_cast<size_t>(r) * a.num_kv_heads * D;
                for (int e = 8 * lane; e < a.num_kv_heads * D; e += 8 * 64)
                {
                    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(const_cast<void*>(a.k_cache)) + dst + e) =
                        *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.k_new) + src + e);
                    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(const_cast<void*>(a.v_cache)) + dst + e) =
                        *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.v_new) + src + e);
                }
            }
        }
        P += w.total;
        if (w.w0 + 64 >= B) break;
        w = load_win(w.w0 + 64, P);
    }
    // Work item i of W takes pages [i * P / W, (i + 1) * P / W), W = min(items, P) so that every item has a page.
    // PW (fused shared-prefix launch): the first pfx_items items also compute prefix partials, so each of them
    // weighs pfx_share / 1024 of another item: pages [P * cum(i) / T, P * cum(i + 1) / T) with cum(i) = 1024 i -
    // min(i, pfx_items) (1024 - pfx_share) and T = cum(items), as long as that still leaves every item a page.
    const int     item = item_of();
    const int     n_items = PW ? n_items_ : static_cast<int>(gridDim.x);
    const int64_t uh = a.pfx_share, up = 1024, H = a.pfx_items;
    const int64_t T_w = H * uh + (n_items - H) * up;
    const bool    weighted = PW && H > 0 && static_cast<int64_t>(P) * min(uh, up) >= T_w;
    const int     W = weighted ? n_items : min(n_items, P);
    if (item >= W) return;
    auto cum = [&](int64_t i) { return i * up - min(i, H) * (up - uh); };
    const int start = weighted ? static_cast<int>(static_cast<int64_t>(P) * cum(item) / T_w)
                               : static_cast<int>(static_cast<int64_t>(item) * P / W);
    const int end = weighted ? static_cast<int>(static_cast<int64_t>(P) * cum(item + 1) / T_w)
                             : static_cast<int>(static_cast<int64_t>(item + 1) * P / W);
    // largest item i with start(i) <= x
    auto last_item = [&](int64_t x) -> int
    {
        if (!weighted) return static_cast<int>(((x + 1) * W + P - 1) / P - 1);  // largest i with i*P/W <= x
        const int64_t K = ((x + 1) * T_w + P - 1) / P - 1;                      // cum(i) <= K
        return static_cast<int>(K < H * uh ? K / uh : H + (K - H * uh) / up);
    };

    // wave -> (KV head, block of 16 of its query heads): heads kvh * G + h0 + c for c < gc
    const int G = a.group;
    const int HB = (G + 15) >> 4;
    const int vh = y_of() * (PW ? nw_ : static_cast<int>(blockDim.x) >> 6) + wave;
    if (vh >= a.num_kv_heads * HB) return;
    const int kvh = vh / HB;
    const int h0 = (vh - kvh * HB) * 16;
    const int gc = min(16, G - h0);  // heads of this block
    uint16_t* sv = s_v + wave * (kBlockSize * D);

    float kv_scale_log2 = a.scale_log2;
    float v_head_scale = 1.0f;
    if constexpr (CT == FP8)
    {
        kv_scale_log2 *= a.k_scale[kvh];
        v_head_scale = a.v_scale[kvh];
    }

    // V chunks of this lane: chunk i = 64 j + lane of the wave's page slice is token row i / VCPR, 16 bytes at
    // (i % VCPR) * 16 of it (VCPR 16-byte chunks a row; rows past the page's 16 are not loaded: 8-bit head_dim 96)
    // (recomputed where used from the lane and the constant j: cheaper than holding them in registers)
    const int     v_row_bytes = a.num_kv_heads * D * kElemBytes<CT>;  // token stride of the pages
    auto          v_tok = [&](int j) { return (64 * j + lane) / VCPR; };
    auto          v_chk = [&](int j) { return (64 * j + lane) % VCPR; };

    // ---- load cursor: the next page to load and its row -----------------------------------------------------
    // The row's block-table entries come 64 at a time (lane l: entry tb + l); the next row with pages, and its
    // first 64 entries, are fetched as soon as the cursor enters a row, so crossing into it costs no round trip.
    struct LRow
    {
        int            b, pb, nb, lp;
        const int32_t* table;
        int            ns;  // fused append: slot of the new token in the row's last page, or -1
    };
    Win  win = win0;  // window of the most advanced row found so far
    auto row_at = [&](int b)  // row b, which lies in `win`
    {
        const int l = b - win.w0;
        const int toks = __builtin_amdgcn_readlane(win.toks, l);
        const int ns = a.k_new != nullptr && toks > 0 && __builtin_amdgcn_readlane(win.whole, l) ? (toks - 1) & 15 : -1;
        return LRow{b, win.base + __builtin_amdgcn_readlane(win.excl, l), __builtin_amdgcn_readlane(win.n, l), toks,
                    a.block_table + static_cast<int64_t>(b) * a.max_blocks + a.skip_blocks, ns};
    };
    auto find_page = [&](int x)  // row holding page x (x < P), moving `win` forward from its current window
    {
        for (;;)
        {
            const uint64_t hit = __ballot(win.w0 + lane < B && win.base + win.excl <= x && x < win.base + win.excl + win.n);
            if (hit != 0) return row_at(win.w0 + __ffsll(static_cast<long long>(hit)) - 1);
            win = load_win(win.w0 + 64, win.base + win.total);
        }
    };
    auto next_row = [&](const LRow& r)  // the next row with pages (one exists)
    {
        for (;;)
        {
            const int      from = r.b + 1 - win.w0;  // lanes at or above `from` are candidates
            const uint64_t m = __ballot(win.w0 + lane < B && win.n > 0 && lane >= from);
            if (m != 0) return row_at(win.w0 + __ffsll(static_cast<long long>(m)) - 1);
            win = load_win(win.w0 + 64, win.base + win.total);
        }
    };
    auto load_tvec = [&](const LRow& r, int tb) { return tb + lane < r.nb ? r.table[tb + lane] : -1; };

    LRow lrow = find_page(start);
    int  tb = (start - lrow.pb) & ~63;
    int  tvec = load_tvec(lrow, tb);
    LRow lnxt = lrow;
    int  ntvec = -1;
    auto look_ahead = [&]()  // fetch the row after lrow if the item reaches it
    {
        if (lrow.pb + lrow.nb < end)
        {
            lnxt = next_row(lrow);
            ntvec = load_tvec(lnxt, 0);
        }
    };
    look_ahead();
    int lp = start;  // next page to load

    // Issue the K and V loads of page lp into r and advance the cursor.
    auto load_next = [&](PageRegs<NW, NWV>& r)
    {
        if (lp == lrow.pb + lrow.nb)
        {
            lrow = lnxt;
            tb = 0;
            tvec = ntvec;
            look_ahead();
        }
        const int pg = lp - lrow.pb;
        if (pg - tb >= 64)
        {
            tb += 64;
            tvec = load_tvec(lrow, tb);
        }
        const int phys = __builtin_amdgcn_readlane(tvec, pg - tb);
        ++lp;
        r.b = lrow.b;
        r.pb = lrow.pb;
        r.nb = lrow.nb;
        r.lp = lrow.lp;
        r.phys = phys;
        r.ok = phys >= 0 && phys < a.num_blocks;  // uniform: a masked page is skipped
        r.ns = pg == lrow.nb - 1 ? lrow.ns : -1;  // fused append: the new token sits in the row's last page
        if (!r.ok) return;
        const size_t row_c = (static_cast<size_t>(phys) * kBlockSize + c) * a.num_kv_heads + kvh;
        if constexpr (CT == I8)
        {
            // issued before the page's K/V: waiting for them never waits for a later load
            r.ks = a.k_scale[row_c];
            r.vs = a.v_scale[row_c];
        }
        // V: whole 16-byte chunks of the slice, rows v_tok (non-temporal)
        const char* vpage = static_cast<const char*>(a.v_cache) +
                            (static_cast<size_t>(phys) * kBlockSize * a.num_kv_heads + kvh) * D * kElemBytes<CT>;
        if constexpr (kElemBytes<CT> == 2)
        {
            const char* kp = static_cast<const char*>(a.k_cache) + row_c * D * 2;
            if (c == r.ns)  // fused append: the new token comes from the step's k / v (same dtype as the cache)
                kp = static_cast<const char*>(a.k_new) + (static_cast<size_t>(lrow.b) * a.num_kv_heads + kvh) * D * 2;
            const char* vnew = static_cast<const char*>(a.v_new) + (static_cast<size_t>(lrow.b) * a.num_kv_heads + kvh) * D * 2;
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j) r.k[j] = load16<FFKV_DECODE_NT_K>(kp + dim_of<CT>(j, g) * 2);
            if constexpr (KT) r.kt = *reinterpret_cast<const u32x2*>(kp + (DT + 4 * g) * 2);
#pragma unroll
            for (int j = 0; j < NWV; ++j)
                r.v[j] = v_tok(j) < kBlockSize
                             ? load16<FFKV_DECODE_NT_V>(v_tok(j) == r.ns
                                                            ? vnew + 16 * v_chk(j)
                                                            : vpage + static_cast<uint32_t>(v_tok(j) * v_row_bytes +
                                                                                            16 * v_chk(j)))
                             : u32x4{0u, 0u, 0u, 0u};
        }
        else
        {
            const char* kp = static_cast<const char*>(a.k_cache) + row_c * D;
#pragma unroll
            for (int j = 0; j < KSTEPS; j += 2)
            {
                if (j + 1 < KSTEPS)
                {
                    r.k[j / 2] = load16<FFKV_DECODE_NT_K>(kp + dimof(j, g));
                }
                else  // an odd last k-step: its 8 codes alone
                {
                    const u32x2 tk = *reinterpret_cast<const u32x2*>(kp + dimof(j, g));
                    r.k[j / 2] = u32x4{tk[0], tk[1], 0u, 0u};
                }
            }
            if constexpr (KT) r.kt = u32x2{*reinterpret_cast<const uint32_t*>(kp + DT + 4 * g), 0u};
#pragma unroll
            for (int j = 0; j < NWV; ++j)
                r.v[j] = v_tok(j) < kBlockSize ? load16<FFKV_DECODE_NT_V>(vpage + static_cast<uint32_t>(v_tok(j) * v_row_bytes + 16 * v_chk(j))) : u32x4{0u, 0u, 0u, 0u};
        }
    };

    X8   qhi[KSTEPS > 0 ? KSTEPS : 1], qlo[KSTEPS > 0 ? KSTEPS : 1];
    X4   qthi, qtlo;  // last 16-dim k-step (KT): dims DT + 4g .. + 3
    auto load_q = [&](int b)  // Q of row b's group as MFMA B operands (column c = head, zero beyond the group)
    {
        if constexpr (KT)
        {
            const size_t e = (static_cast<size_t>(b) * a.num_heads + kvh * G + h0 + c) * D + DT + 4 * g;
            float        x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (c < gc)
            {
                if constexpr (QT == F32)
                {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.q) + e);
#pragma unroll
                    for (int i = 0; i < 4; ++i) x[i] = v[i];
                }
                else
                {
                    const u32x2 w = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(a.q) + e);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                    {
                        const uint32_t h = (w[i >> 1] >> (16 * (i & 1))) & 0xffffu;
                        x[i] = QT == BF16 ? bf16_to_f32(h) : f16_to_f32(h);
                    }
                }
            }
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                hi[i] = M::bits(x[i]);
                lo[i] = NEED_LO ? M::bits(x[i] - M::value(hi[i])) : 0u;
            }
            qthi = __builtin_bit_cast(X4, u32x2{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)});
            qtlo = __builtin_bit_cast(X4, u32x2{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)});
        }
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
            if constexpr (!NEED_LO)
            {
                // q is stored in the MFMA input type: its 16 bytes are the operand
                u32x4 w = u32x4{0u, 0u, 0u, 0u};
                if (c < gc)
                    w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.q) +
                                                        (static_cast<size_t>(b) * a.num_heads + kvh * G + h0 + c) * D +
                                                        dimof(j, g));
                qhi[j] = __builtin_bit_cast(X8, w);
                qlo[j] = qhi[j];
            }
            else
            {
                float x[8];
                if (c < gc)
                    load_q8<QT>(a.q, (static_cast<size_t>(b) * a.num_heads + kvh * G + h0 + c) * D + dimof(j, g),
                                x);
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

    // K or V words of k-step j in the MFMA input type.
    // k-step j's 8 values as MFMA words: of type bf16 (TBF) or f16 for 8-bit codes
    auto mword = [&]<bool TBF>(const u32x4* w, int j) -> u32x4
    {
        if constexpr (kElemBytes<CT> == 2)
            return w[j];
        else
            return (j & 1) ? codes_to_m<CT, TBF>(w[j / 2][2], w[j / 2][3])
                           : codes_to_m<CT, TBF>(w[j / 2][0], w[j / 2][1]);
    };

    // Stage a loaded page: V rows into the wave's LDS tile, scores S^T = K Q^T into s.  Consumes r.k and r.v,
    // so the next page can be loaded into r right after.
    auto stage_page = [&](int n_tok, const PageRegs<NW, NWV>& r, f32x4& s)
    {
        if constexpr (kElemBytes<CT> == 2)
        {
            // fused append: write the new token's row into its page slot (as ffkv_append)
            if (r.ns >= 0 && h0 == 0)
            {
                const size_t row_n = (static_cast<size_t>(r.phys) * kBlockSize + r.ns) * a.num_kv_heads + kvh;
                char*        kp = static_cast<char*>(const_cast<void*>(a.k_cache)) + row_n * D * 2;
                char*        vp = static_cast<char*>(const_cast<void*>(a.v_cache)) + row_n * D * 2;
                if (c == r.ns)
                {
#pragma unroll
                    for (int j = 0; j < KSTEPS; ++j) *reinterpret_cast<u32x4*>(kp + dim_of<CT>(j, g) * 2) = r.k[j];
                    if constexpr (KT) *reinterpret_cast<u32x2*>(kp + (DT + 4 * g) * 2) = r.kt;
                }
#pragma unroll
                for (int j = 0; j < NWV; ++j)
                    if (v_tok(j) == r.ns) *reinterpret_cast<u32x4*>(vp + 16 * v_chk(j)) = r.v[j];
            }
        }
        // V rows into the LDS tile, zero for slots past the row's last token (chunks past the page's 16 rows:
        // head_dim 80 and 112, and 8-bit 96, whose pages fill the last load instruction in part)
#pragma unroll
        for (int j = 0; j < NWV; ++j)
        {
            const int  t = v_tok(j);
            const bool tok_ok = t < n_tok;
            if (t >= kBlockSize) continue;
            if constexpr (kElemBytes<CT> == 2)
            {
                const u32x4 w = tok_ok ? r.v[j] : u32x4{0u, 0u, 0u, 0u};
                *reinterpret_cast<u32x4*>(sv + vt_pos<D>(t, 8 * v_chk(j))) = w;
            }
            else  // 16 codes: dims 16 ch .. 16 ch + 15 as two 8-value words
            {
                const u32x4 lo = tok_ok ? codes_to_m<CT, VBF>(r.v[j][0], r.v[j][1]) : u32x4{0u, 0u, 0u, 0u};
                const u32x4 hi = tok_ok ? codes_to_m<CT, VBF>(r.v[j][2], r.v[j][3]) : u32x4{0u, 0u, 0u, 0u};
                *reinterpret_cast<u32x4*>(sv + vt_pos<D>(t, 16 * v_chk(j))) = lo;
                *reinterpret_cast<u32x4*>(sv + vt_pos<D>(t, 16 * v_chk(j) + 8)) = hi;
            }
        }
        s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};  // lane (c, g) gets tokens 4g + i of head c
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j)
        {
            const X8 kj = __builtin_bit_cast(X8, mword.template operator()<BF>(r.k, j));
            s = M::mma32(kj, qhi[j], s);
            if constexpr (NEED_LO) s = M::mma32(kj, qlo[j], s);
        }
        if constexpr (KT)  // the last 16 dims: 4 per lane
        {
            u32x2 w = r.kt;
            if constexpr (kElemBytes<CT> == 1)
            {
                const u32x4 m = codes_to_m<CT, BF>(r.kt[0], 0u);
                w = u32x2{m[0], m[1]};
            }
            // Its products accumulate apart and join the scores by vector adds: a 16x16x16 product that takes the
            // 16x16x32 chain's result as its accumulator input got no wait states between them from this compiler
            // (gfx950), and read the accumulator before the chain had written it (the scores of head_dim 80 and 112
            // lost their first 64 or 96 dims on the GPU).
            const X4 kt = __builtin_bit_cast(X4, w);
            f32x4    st = M::mma16(kt, qthi, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
            if constexpr (NEED_LO) st = M::mma16(kt, qtlo, st);
            s += st;
        }
    };

    // Online softmax of a staged page's scores and PV from its LDS tile.  tks / tvs: int8 scales of token c.
    auto finish_page = [&](int n_tok, float tks, float tvs, f32x4 s)
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
            for (int i = 0; i < 4; ++i)  // token 4g + i's scales sit in lane 4g + i
            {
                ks[i] = __shfl(tks, 4 * g + i, 64);
                vs[i] = __shfl(tvs, 4 * g + i, 64);
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

        // P^T as MFMA B operands (k = token 4g + i, column c = head); bf16 P as hi + lo parts
        uint32_t ph[4], pl[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            ph[i] = MV::bits(pv[i]);
            pl[i] = P_LO ? MV::bits(pv[i] - MV::value(ph[i])) : 0u;
        }
        const typename MV::x4 phi =
            __builtin_bit_cast(typename MV::x4, u32x2{ph[0] | (ph[1] << 16), ph[2] | (ph[3] << 16)});
        const typename MV::x4 plo =
            __builtin_bit_cast(typename MV::x4, u32x2{pl[0] | (pl[1] << 16), pl[2] | (pl[3] << 16)});

        // LDS writes of this wave are complete before its reads below (in-order LDS queue of one wave);
        // the fence keeps the compiler from moving the reads above the writes.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // O^T[d, h] += V^T[d, t] P^T[t, h] over the 16 dims of each tile
#pragma unroll
        for (int n = 0; n < NT; ++n)
        {
            // transposed read: lane 4r + q of group g supplies dims 16n + 4q .. +3 of token 4g + r; lane c
            // receives dim 16n + c of tokens 4g .. 4g + 3
            const auto raw = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                (__attribute__((address_space(3))) bf16x4*)(sv + vt_pos<D>(4 * g + (c >> 2), 16 * n + 4 * (c & 3))));
            const typename MV::x4 vt = __builtin_bit_cast(typename MV::x4, raw);
            acc[n] = MV::mma16(vt, phi, acc[n]);
            if constexpr (P_LO) acc[n] = MV::mma16(vt, plo, acc[n]);
        }
        // the next page's LDS writes must not overtake these reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // Write the segment [seg_start, seg_end) of row b (pages pb .. pb + nb - 1): the output if it is the whole row,
    // else a partial.
    auto finish_segment = [&](int b, int pb, int nb, int seg_start, int seg_end)
    {
        const float l_tot = xor_sum(l_run);
        const int   h = kvh * G + h0 + c;
        if (seg_start == pb && seg_end == pb + nb && a.pfx_chunks == 0)
        {
            if (c < gc)
            {
                const float inv = l_tot > 0.0f ? v_head_scale / l_tot : 0.0f;
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    store_out4<QT>(a.out, (static_cast<size_t>(b) * a.num_heads + h) * D + 16 * n + 4 * g,
                                   acc[n] * inv);
            }
        }
        else if (c < gc)
        {
            const int64_t slot = static_cast<int64_t>(item) + b;
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
        if (seg_start == pb && y_of() == 0 && wave == 0 && lane == 0)
        {
            a.ws_meta[2 * b] = item;
            a.ws_meta[2 * b + 1] = last_item(pb + nb - 1);
        }
    };

    // ---- pages start .. end - 1, DEPTH of them in flight ---------------------------------------------------
    // Page p sits in r[(p - start) % DEPTH]; right after it is staged, page p + DEPTH is loaded into the same
    // registers, and stays in flight while p is finished.
    load_q(lrow.b);
    int seg_start = start;
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    PageRegs<NW, NWV> r[DEPTH];
#pragma unroll
    for (int sl = 0; sl < DEPTH; ++sl)
        if (start + sl < end) load_next(r[sl]);

    auto step = [&]<int S>(int p)
    {
        PageRegs<NW, NWV>& cur = r[S];
        const int     b = cur.b, pb = cur.pb, nb = cur.nb;
        const float   tks = cur.ks, tvs = cur.vs;
        const bool    ok = cur.ok;
        const int     n_tok = min(kBlockSize, cur.lp - (p - pb) * kBlockSize);
        const bool    row_ends = p + 1 == pb + nb;
        f32x4         s;
        if (ok) stage_page(n_tok, cur, s);
        // The scores of page p have consumed Q: a new row's Q is loaded now, ahead of page p + DEPTH's K/V when
        // page p + 1 is already in flight (loads complete in issue order for the wait counter).
        if constexpr (DEPTH > 1)
            if (row_ends && p + 1 < end) load_q(r[(S + 1) % DEPTH].b);
        if (p + DEPTH < end) load_next(cur);
        if constexpr (DEPTH == 1)
            if (row_ends && p + 1 < end) load_q(cur.b);
        if (ok) finish_page(n_tok, tks, tvs, s);
        if (row_ends || p + 1 == end)
        {
            finish_segment(b, pb, nb, seg_start, p + 1);
            seg_start = p + 1;
            m_run = kNegInf;
            l_run = 0.0f;
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    for (int p = start; p < end; p += DEPTH)
    {
        step.template operator()<0>(p);
        if constexpr (DEPTH > 1)
            if (p + 1 < end) step.template operator()<1 % DEPTH>(p + 1);
        if constexpr (DEPTH > 2)
            if (p + 2 < end) step.template operator()<2 % DEPTH>(p + 2);
    }
}

#if FFKV_DECODE_TIMELINE
// Timeline builds: wave w of a launch (w = (blockIdx.y * gridDim.x + blockIdx.x) * NW + wave) records its start
// and end on the GPU's constant 100 MHz clock in entries 2w and 2w + 1; ffkv_decode_timeline reads them back.
constexpr int kTimelineWaves = 1 << 16;
static __device__ uint64_t g_decode_timeline[2 * kTimelineWaves];
#endif

// Work item blockIdx.x of gridDim.x; KV heads blockIdx.y * NW .. +NW, one per wave (NW = blockDim.x / 64).
template <int CT, int QT, int D>
__global__ __launch_bounds__((64 * kMfmaMaxWaves<CT, D>)) __attribute__((amdgpu_waves_per_eu(kMfmaWaves<CT, QT, D>, 8)))
void paged_decode_mfma(DecodeArgs a)
{
    __shared__ uint16_t s_v[kMfmaMaxWaves<CT, D> * kBlockSize * D];
#if FFKV_DECODE_TIMELINE
    const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
#endif
    decode_wg<CT, QT, D>(a, static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y), static_cast<int>(gridDim.x),
                         static_cast<int>(blockDim.x) >> 6, s_v);
#if FFKV_DECODE_TIMELINE
    const uint64_t t_end = __builtin_amdgcn_s_memrealtime();
    const int      lane = static_cast<int>(threadIdx.x) & 63;
    const int      w = (static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x) * static_cast<int>(blockDim.x >> 6)) +
                  (static_cast<int>(threadIdx.x) >> 6);
    if (lane < 2 && w < kTimelineWaves)  // two lanes, one vector store each
        g_decode_timeline[2 * w + lane] = lane == 0 ? t_start : t_end;
#endif
}

// Combine the partials of rows split over several work items.
// One workgroup of four waves per (row, head): wave w folds segments i_lo + w, i_lo + w + 4, ... into an online
// (max, denominator, output) state (lane = D/64 dims), then the four states are combined through LDS.
// MW waves per (row, head): 4 for short piece lists, 16 when rows are few and long (C3-like) and each row has
// tens of pieces.
template <int QT, int D, int MW>
__global__ __launch_bounds__(64 * MW) void paged_decode_mfma_merge(DecodeArgs a)
{
    constexpr int PER = (D + 63) / 64;  // dims per lane (head_dim 96: lanes 0 .. 47 hold two)
    const int     b = blockIdx.x;
    const int     h = blockIdx.y;
    const int     lane = threadIdx.x & 63;
    const int     wave = threadIdx.x >> 6;
    const size_t  ob = (static_cast<size_t>(b) * a.num_heads + h) * D;
    __shared__ float s_m[MW], s_l[MW];
    __shared__ float s_o[MW][D];

    const int i_lo = a.ws_meta[2 * b];
    const int i_hi = a.ws_meta[2 * b + 1];
    // one piece (written by the decode kernel) or no token (i_lo = i_hi = -1); shared-prefix mode always merges
    if (i_lo == i_hi && a.pfx_chunks == 0) return;

    // pieces: the shared-prefix partials (slots pfx_slot0 + k * batch + b), then work items i_lo .. i_hi (slots
    // i + b) when the row has pages of its own
    const int pieces = a.pfx_chunks + (i_lo >= 0 ? i_hi - i_lo + 1 : 0);
    float     m = kNegInf, l = 0.0f, o[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) o[k] = 0.0f;
    // Wave w folds pieces w, w + MW, ...; the loads of FOLD pieces go out together before any is folded, so a
    // row of up to MW * FOLD pieces costs one round trip to memory instead of one per piece.
    constexpr int FOLD = 4;
    for (int i0 = wave; i0 < pieces; i0 += MW * FOLD)
    {
        float ms[FOLD], ls[FOLD], x[FOLD][PER];
#pragma unroll
        for (int f = 0; f < FOLD; ++f)
        {
            const int i = i0 + MW * f;
            ms[f] = kNegInf;
            ls[f] = 0.0f;
#pragma unroll
            for (int k = 0; k < PER; ++k) x[f][k] = 0.0f;
            if (i < pieces)
            {
                const int64_t slot = i < a.pfx_chunks
                                         ? static_cast<int64_t>(a.pfx_slot0) + static_cast<int64_t>(i) * a.batch + b
                                         : static_cast<int64_t>(i_lo + i - a.pfx_chunks) + b;
                ms[f] = a.ws_ml[(slot * a.num_heads + h) * 2];
                ls[f] = a.ws_ml[(slot * a.num_heads + h) * 2 + 1];
                const float* src = a.ws_acc + (slot * a.num_heads + h) * D + lane * PER;
#pragma unroll
                for (int k = 0; k < PER; ++k) x[f][k] = lane * PER + k < D ? src[k] : 0.0f;
            }
        }
#pragma unroll
        for (int f = 0; f < FOLD; ++f)
        {
            if (ms[f] == kNegInf) continue;  // segment without a valid page (or past the row's pieces)
            const float mn = fmaxf(m, ms[f]);
            const float wa = __builtin_amdgcn_exp2f(m - mn);
            const float wb = __builtin_amdgcn_exp2f(ms[f] - mn);
            l = l * wa + ls[f] * wb;
#pragma unroll
            for (int k = 0; k < PER; ++k) o[k] = o[k] * wa + x[f][k] * wb;
            m = mn;
        }
    }
    if (lane == 0)
    {
        s_m[wave] = m;
        s_l[wave] = l;
    }
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (lane * PER + k < D) s_o[wave][lane * PER + k] = o[k];
    __syncthreads();
    if (threadIdx.x < D)
    {
        const int d = threadIdx.x;
        float     M = kNegInf;
#pragma unroll
        for (int w = 0; w < MW; ++w) M = fmaxf(M, s_m[w]);
        float L = 0.0f, O = 0.0f;
        if (M != kNegInf)
        {
#pragma unroll
            for (int w = 0; w < MW; ++w)
            {
                const float wt = __builtin_amdgcn_exp2f(s_m[w] - M);
                L += s_l[w] * wt;
                O += s_o[w][d] * wt;
            }
        }
        store_act1(a.out, QT, ob + d, L > 0.0f ? O / L : 0.0f);
    }
}

// Combine the partials of split rows when each row has few pieces (more than 16 rows): thread k of the row's
// workgroups owns output dims 4(k % (D/4)) .. +3 of head k / (D/4), folds that chunk of every piece of the row
// (loads of up to MF = 16 pieces in flight together) and writes it; no cross-thread combine.  Rows written whole by
// the decode kernel (one piece, no shared-prefix partials) or without tokens are left alone.
template <int QT, int D>
__global__ __launch_bounds__(256) void paged_decode_mfma_merge_rows(DecodeArgs a)
{
    constexpr int MF = 16;
    const int     b = blockIdx.x;
    const int     k = static_cast<int>(blockIdx.y) * 256 + static_cast<int>(threadIdx.x);
    const int     i_lo = a.ws_meta[2 * b];
    const int     i_hi = a.ws_meta[2 * b + 1];
    if ((i_lo == i_hi && a.pfx_chunks == 0) || k >= a.num_heads * (D / 4)) return;
    const int     h = k / (D / 4);
    const int     d4 = (k - h * (D / 4)) * 4;
    const int     pieces = a.pfx_chunks + (i_lo >= 0 ? i_hi - i_lo + 1 : 0);
    float         m = kNegInf, l = 0.0f;
    f32x4         o = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int i0 = 0; i0 < pieces; i0 += MF)
    {
        float ms[MF], ls[MF];
        f32x4 xs[MF];
#pragma unroll
        for (int f = 0; f < MF; ++f)
        {
            ms[f] = kNegInf;
            ls[f] = 0.0f;
            xs[f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            const int i = i0 + f;
            if (i < pieces)
            {
                // the shared-prefix partials (slots pfx_slot0 + j * batch + b), then work items i_lo .. i_hi (slots
                // item + b)
                const int64_t slot = i < a.pfx_chunks
                                         ? static_cast<int64_t>(a.pfx_slot0) + static_cast<int64_t>(i) * a.batch + b
                                         : static_cast<int64_t>(i_lo + i - a.pfx_chunks) + b;
                const int64_t e = slot * a.num_heads + h;
                const float2  ml = *reinterpret_cast<const float2*>(a.ws_ml + e * 2);
                ms[f] = ml.x;
                ls[f] = ml.y;
                xs[f] = *reinterpret_cast<const f32x4*>(a.ws_acc + e * D + d4);
            }
        }
#pragma unroll
        for (int f = 0; f < MF; ++f)
        {
            if (ms[f] == kNegInf) continue;  // a piece without a valid page (or past the row's pieces)
            const float mn = fmaxf(m, ms[f]);
            const float wa = __builtin_amdgcn_exp2f(m - mn);
            const float wb = __builtin_amdgcn_exp2f(ms[f] - mn);
            l = l * wa + ls[f] * wb;
            o = o * wa + xs[f] * wb;
            m = mn;
        }
    }
    store_out4<QT>(a.out, (static_cast<size_t>(b) * a.num_heads + h) * D + d4,
                   l > 0.0f ? o * (1.0f / l) : f32x4{0.0f, 0.0f, 0.0f, 0.0f});
}

namespace
{

// Waves per workgroup and workgroups per work item (grid y) of a launch: one wave per KV head and block of 16
// query heads, up to kMfmaMaxWaves per workgroup.
struct MfmaShape
{
    int nw, gy;
};

template <int CT, int D>
MfmaShape mfma_shape(const DecodeArgs& a)
{
    const int vh = a.num_kv_heads * ((a.group + 15) / 16);
    const int nw = vh < kMfmaMaxWaves<CT, D> ? vh : kMfmaMaxWaves<CT, D>;
    return MfmaShape{nw, (vh + nw - 1) / nw};
}

template <int CT, int QT, int D>
int items_m3(const DecodeArgs& a)
{
    const MfmaShape sh = mfma_shape<CT, D>(a);
    return decode_mfma_items(reinterpret_cast<const void*>(paged_decode_mfma<CT, QT, D>), 64 * sh.nw, sh.gy);
}

// The merge after a decode launch (rows split over several items, or shared-prefix partials).
template <int QT, int D>
hipError_t launch_merge(const DecodeArgs& a, hipStream_t stream)
{
    if (a.batch <= FFKV_MERGE_ROWS_MIN_BATCH)  // few rows over the same items: tens of pieces per row
    {
        const dim3 mgrid(static_cast<unsigned>(a.batch), static_cast<unsigned>(a.num_heads));
        hipLaunchKernelGGL((paged_decode_mfma_merge<QT, D, 16>), mgrid, dim3(1024), 0, stream, a);
    }
    else
    {
        const dim3 mgrid(static_cast<unsigned>(a.batch), static_cast<unsigned>((a.num_heads * (D / 4) + 255) / 256));
        hipLaunchKernelGGL((paged_decode_mfma_merge_rows<QT, D>), mgrid, dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

template <int CT, int QT, int D>
hipError_t launch_m3(const DecodeArgs& a, hipStream_t stream)
{
    const MfmaShape sh = mfma_shape<CT, D>(a);
    const int       nw = sh.nw, gy = sh.gy;
    const auto      kern = paged_decode_mfma<CT, QT, D>;
    // the workspace holds items + batch partial slots
    const int items = a.items > 0 ? a.items : items_m3<CT, QT, D>(a);
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(items), static_cast<unsigned>(gy)), dim3(64 * nw), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_merge<QT, D>(a, stream);
}

template <int CT, int QT>
int items_m2(const DecodeArgs& a)
{
    switch (a.head_dim)
    {
        case 64:
            return items_m3<CT, QT, 64>(a);
        case 80:
            return items_m3<CT, QT, 80>(a);
        case 96:
            return items_m3<CT, QT, 96>(a);
        case 112:
            return items_m3<CT, QT, 112>(a);
        case 128:
            return items_m3<CT, QT, 128>(a);
        default:
            return items_m3<CT, QT, 256>(a);
    }
}

template <int CT>
int items_m1(const DecodeArgs& a)
{
    switch (a.qo_dtype)
    {
        case F32:
            return items_m2<CT, F32>(a);
        case F16:
            return items_m2<CT, F16>(a);
        default:
            return items_m2<CT, BF16>(a);
    }
}

template <int CT, int QT>
hipError_t launch_m2(const DecodeArgs& a, hipStream_t stream)
{
    switch (a.head_dim)
    {
        case 64:
            return launch_m3<CT, QT, 64>(a, stream);
        case 80:
            return launch_m3<CT, QT, 80>(a, stream);
        case 96:
            return launch_m3<CT, QT, 96>(a, stream);
        case 112:
            return launch_m3<CT, QT, 112>(a, stream);
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

#ifndef FFKV_DEVICE_BODIES_ONLY

int decode_mfma_launch_items(const DecodeArgs& a)
{
    switch (a.cache_dtype)
    {
        case BF16:
            return items_m1<BF16>(a);
        case F16:
            return items_m1<F16>(a);
        case I8:
            return items_m1<I8>(a);
        default:
            return items_m1<FP8>(a);
    }
}

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

#endif  // FFKV_DEVICE_BODIES_ONLY

}  // namespace ffkv

#if FFKV_DECODE_TIMELINE && !defined(FFKV_DEVICE_BODIES_ONLY)
// Timeline builds only (python -m firefly_amd.build --define FFKV_DECODE_TIMELINE=1 --out ...; bench.py --timeline):
// clear != 0 zeroes the record, else up to max_waves (start, end) pairs of the last split-K launches are copied to
// out (2 * max_waves values, 100 MHz clock ticks; waves that recorded nothing read 0).  Synchronous.
extern "C" __attribute__((visibility("default"))) int ffkv_decode_timeline(uint64_t* out, int max_waves, int clear)
{
    const size_t n = static_cast<size_t>(max_waves < ffkv::kTimelineWaves ? max_waves : ffkv::kTimelineWaves);
    void*        p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(ffkv::g_decode_timeline)) != hipSuccess) return -1;
    if (clear != 0) return hipMemset(p, 0, sizeof(ffkv::g_decode_timeline)) == hipSuccess ? 0 : -1;
    if (out == nullptr || max_waves <= 0) return -1;
    return hipMemcpy(out, p, 2 * n * sizeof(uint64_t), hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif
